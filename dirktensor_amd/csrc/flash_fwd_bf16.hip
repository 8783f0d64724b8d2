// Causal flash attention forward, bf16 MFMA mode, for gfx950 (CDNA4).
//
// Replaces flash_attention_forward (FlashAttention.cpp:24-182) with bf16
// Q/K/V/O, fp32 accumulation and an fp32 online softmax.
//
// Work decomposition
//   * An item is 128 queries of one (batch, head). A persistent grid of at most
//     one workgroup per CU walks the items in "snake" order over a list sorted
//     by causal cost (item k of round j: j*G + w on even rounds, (j+1)*G-1-w on
//     odd ones), so a workgroup pairs a long query tile with a short one; at
//     T = 4096, H = 16 every workgroup gets 33 key tiles of work.
//   * A workgroup has 8 waves in two groups of 4. Both groups hold the same 128
//     queries (32 per wave) and split the key tiles: group g takes 64-key tiles
//     g, g+2, g+4, ... Each group streams its tiles through its own pair of LDS
//     buffers (double buffering, one barrier per step). At the end group 1
//     hands its partial (max, sum, O) to group 0 through LDS and group 0 merges
//     them with the same rescale the reference applies between tiles
//     (FlashAttention.cpp:134-156).
//   * Within a wave, S^T = K Q^T comes from v_mfma_f32_32x32x16_bf16 with K
//     rows from LDS as the A operand and the wave's Q fragment, held in
//     registers, as B; one lane then owns one query and 16 keys per 32-key
//     block, so the row max and row sum are a per-lane reduction plus one
//     exchange between the lane halves. P is converted to bf16 in registers
//     and used as the B operand of O^T += V^T P^T; the A operand (V^T) comes from the gfx950
//     transposing LDS read ds_read_b64_tr_b16, where a 16-lane group reads a
//     4-key x 16-dim block and each lane receives one dim column of 4 keys,
//     i.e. the MFMA's 8-key k slice taken as two 4-key runs in the
//     accumulator's key order.
//
// Softmax bookkeeping, per query, in the log2 domain of the scaled score
// s' = (scale * log2 e) * q.k (Q is pre-multiplied by scale * log2 e when its
// fragment is loaded):
//   m_t  running true maximum of s' (the reference's m is m_t / log2 e);
//   m_s  the maximum the probabilities are currently taken relative to. The S
//        MFMA chain starts from the accumulator -m_s, so it yields t = s' - m_s
//        directly and p = exp2(t) needs no further arithmetic. m_s is raised
//        to m_t only when some t of the wave exceeds 8 (p would exceed 2^8),
//        so O and l are rescaled rarely; at the end l is reported relative to
//        m_t: l = sum exp(s - m) = l_s * exp2(m_s - m_t).
//   l    the row sum of the bf16 probabilities that enter the PV product,
//        accumulated with v_dot2 against (1, 1).
// Keys with k_pos > q_pos are masked (FlashAttention.cpp:102); a row with no
// valid key is written as the reference's empty row (FlashAttention.cpp:165-174).
// K and V tiles are read with buffer loads whose descriptor ends at the
// sequence's last valid key, so rows past it load as zeros without branches.

#include "dt_internal.h"

namespace dt {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef short shortx8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;
typedef int intx4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kBM = 128;       // queries per item
constexpr int kBN = 64;        // keys per tile
constexpr int kThreads = 512;  // 8 waves
constexpr int kLdK = 136;      // bf16 elements per K row in LDS (272 B: b128 row reads hit distinct banks)
constexpr int kLdV = 160;      // bf16 elements per V row in LDS (320 B: transposing reads hit distinct banks)
constexpr int kStage = kBN * kLdK + kBN * kLdV;  // bf16 elements per (K, V) stage
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kRescaleLog2 = 8.0f;
constexpr int kBufferDword3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 r = __builtin_convertvector((floatx2){lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, r);
}

// Row reductions across the two lane halves (lane l and lane l ^ 32 hold the same
// query). ds_bpermute via __shfl_xor; v_permlane32_swap would avoid the LDS
// crossbar, but this compiler returns the same register for both of the
// builtin's results, so its second half is unusable.
__device__ __forceinline__ float max_halves(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }
__device__ __forceinline__ float sum_halves(float x) { return x + __shfl_xor(x, 32, 64); }

__device__ __forceinline__ shortx4 lds_read_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(p));
}

// Buffer descriptor over [base, base + bytes): loads at or past the end return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferDword3);
}
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    const intx4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0);
    return __builtin_bit_cast(uint4, v);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

struct Item {
    int b, h, qt;
};

__device__ __forceinline__ Item decode_item(int k, int n_qt, int BH, int H) {
    Item it;
    it.qt = n_qt - 1 - k / BH;  // items sorted by decreasing causal cost
    const int r = k % BH;
    it.b = r / H;
    it.h = r % H;
    return it;
}

__global__ __launch_bounds__(kThreads, 1) void flash_fwd_bf16_kernel(FlashArgs a, SeqLens lens) {
    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * 2 * kStage];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int grp = wave >> 2;  // key-tile group
    const int wq = wave & 3;    // 32-query block within the item
    const int ln = lane & 31;
    const int hh = lane >> 5;
    const int gt = tid & 255;  // thread index within the group
    const int ld_row = gt >> 4;
    const int ld_col = 8 * (gt & 15);
    const int tr_row = (lane & 15) >> 2;
    const int tr_col = 4 * (lane & 3) + 16 * ((lane >> 4) & 1);
    // byte offsets of this thread's four 16-byte chunks within a K/V tile (K and V share the row stride)
    uint32_t voff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) voff[i] = (uint32_t)(((ld_row + 16 * i) * a.ldk + ld_col) * 2);

    const int T = a.T;
    const int n_qt = (T + kBM - 1) / kBM;
    const int BH = a.B * a.H;
    const int n_items = n_qt * BH;
    const int G = gridDim.x;
    const float c = a.scale * kLog2e;

    uint16_t* const stage_base = smem + grp * 2 * kStage;

    for (int round = 0;; ++round) {
        const int k_item = (round & 1) ? (round + 1) * G - 1 - (int)blockIdx.x : round * G + (int)blockIdx.x;
        if (k_item >= n_items) break;
        const Item itm = decode_item(k_item, n_qt, BH, a.H);
        const int b = itm.b, h = itm.h;
        const int L = a.ragged ? lens.len[b] : T;
        const int q0 = itm.qt * kBM;
        const int qw0 = q0 + wq * 32;
        const int qrow = qw0 + ln;

        const uint16_t* Qg = static_cast<const uint16_t*>(a.q) + (int64_t)b * T * a.ldq + (int64_t)h * kD;
        const uint16_t* Kg = static_cast<const uint16_t*>(a.k) + (int64_t)b * T * a.ldk + (int64_t)h * kD;
        const uint16_t* Vg = static_cast<const uint16_t*>(a.v) + (int64_t)b * T * a.ldv + (int64_t)h * kD;
        uint16_t* Og = static_cast<uint16_t*>(a.o) + (int64_t)b * T * a.ldo + (int64_t)h * kD;
        const int64_t stat_base = ((int64_t)b * T) * a.H + h;

        if (q0 >= L) {  // all 128 rows are padding: the reference's empty row
            if (grp == 0 && qrow < T) {
                const uint4 z = make_uint4(0, 0, 0, 0);
                for (int j = 0; j < 8; ++j)
                    *reinterpret_cast<uint4*>(&Og[(int64_t)qrow * a.ldo + 64 * hh + 8 * j]) = z;
                if (hh == 0) {
                    if (a.m) a.m[stat_base + (int64_t)qrow * a.H] = kNegInf;
                    if (a.l) a.l[stat_base + (int64_t)qrow * a.H] = 0.0f;
                }
            }
            continue;  // no LDS was touched: no barrier needed
        }

        // Q fragment: qf[cc] = Q[qrow][16*cc + 8*hh .. +8] (B operand of S^T = K Q^T)
        // Q fragment, pre-multiplied by scale * log2 e: qf[cc] = Q[qrow][16*cc + 8*hh .. +8] * c
        bf16x8 qf[8];
        if (qrow < T) {
            const uint16_t* qp = Qg + (int64_t)qrow * a.ldq + 8 * hh;
#pragma unroll
            for (int cc = 0; cc < 8; ++cc) {
                const uint4 raw = *reinterpret_cast<const uint4*>(qp + 16 * cc);
                const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
                uint32_t sw[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) sw[e] = pack_bf16x2(bf16_lo(w[e]) * c, bf16_hi(w[e]) * c);
                qf[cc] = __builtin_bit_cast(bf16x8, make_uint4(sw[0], sw[1], sw[2], sw[3]));
            }
        } else {
#pragma unroll
            for (int cc = 0; cc < 8; ++cc) qf[cc] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
        }

        floatx16 o[4];
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
        float m_t = kNegInf, m_s = kNegInf, l_run = 0.0f;
        floatx16 neg_ms;  // -m_s (0 while m_s is -inf), the starting accumulator of the S chain
#pragma unroll
        for (int i = 0; i < 16; ++i) neg_ms[i] = 0.0f;

        const int k_end = a.causal ? min(q0 + kBM, L) : L;
        const int n_tiles = (k_end + kBN - 1) / kBN;
        const int n_iter = (n_tiles + 1) / 2;

        uint4 pk_k[4], pk_v[4];
        auto fetch = [&](int k0) {
            const uint32_t bytes = (uint32_t)(L - k0) * (uint32_t)a.ldk * 2u;  // rows k0 .. L-1
            const __amdgpu_buffer_rsrc_t rk = make_rsrc(Kg + (int64_t)k0 * a.ldk, bytes);
            const __amdgpu_buffer_rsrc_t rv = make_rsrc(Vg + (int64_t)k0 * a.ldk, bytes);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pk_k[i] = buffer_load16(rk, voff[i]);
                pk_v[i] = buffer_load16(rv, voff[i]);
            }
        };
        auto stash = [&](uint16_t* st) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                *reinterpret_cast<uint4*>(&st[(ld_row + 16 * i) * kLdK + ld_col]) = pk_k[i];
                *reinterpret_cast<uint4*>(&st[kBN * kLdK + (ld_row + 16 * i) * kLdV + ld_col]) = pk_v[i];
            }
        };

        if (grp < n_tiles) fetch(grp * kBN);
        stash(stage_base);
        __syncthreads();

        for (int it = 0; it < n_iter; ++it) {
            const int kt = 2 * it + grp;
            const int kt_next = kt + 2;
            if (kt_next < n_tiles) fetch(kt_next * kBN);
            const uint16_t* Ks = stage_base + (it & 1) * kStage;
            const uint16_t* Vs = Ks + kBN * kLdK;
            const int k0 = kt * kBN;

            if (kt < n_tiles && !(a.causal && k0 > qw0 + 31)) {
                // t = s' - m_s: the chain starts from -m_s
                floatx16 st[2];
#pragma unroll
                for (int cc = 0; cc < 8; ++cc)
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb) {
                        const bf16x8 kf = __builtin_bit_cast(
                            bf16x8, *reinterpret_cast<const uint4*>(&Ks[(32 * kb + ln) * kLdK + 16 * cc + 8 * hh]));
                        st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[cc], cc == 0 ? neg_ms : st[kb], 0, 0,
                                                                          0);
                    }

                // diagonal / ragged-tail tiles: mask with selects (no per-element branches)
                if ((a.causal && k0 + kBN - 1 > qw0) || k0 + kBN > L) {
                    const int lim = a.causal ? min(qrow, L - 1) : L - 1;  // keys > lim are masked
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const int key = k0 + 32 * kb + 8 * (i / 4) + 4 * hh + (i % 4);
                            st[kb][i] = key > lim ? kNegInf : st[kb][i];
                        }
                }
                float tmax = kNegInf;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, st[kb][i]);
                tmax = max_halves(tmax);
                const float base = (m_s == kNegInf) ? 0.0f : m_s;  // what the chain subtracted
                m_t = fmaxf(m_t, tmax + base);
                const bool grow = (m_s == kNegInf) ? (tmax > kNegInf) : (tmax > kRescaleLog2);
                if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // wave-uniform, rare after the first tile
                    const float m_new = m_t;
                    const float delta = (m_new == kNegInf) ? 0.0f : m_new - base;
                    const float alpha = (m_s == kNegInf) ? 0.0f : exp2f(m_s - m_new);
                    m_s = m_new;
                    l_run *= alpha;
#pragma unroll
                    for (int db = 0; db < 4; ++db)
#pragma unroll
                        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                        for (int i = 0; i < 16; ++i) st[kb][i] -= delta;
                    const float nm = (m_s == kNegInf) ? 0.0f : -m_s;
#pragma unroll
                    for (int i = 0; i < 16; ++i) neg_ms[i] = nm;
                }
                // p = exp2(t) in bf16; the row sum is taken over the bf16 values the PV product uses
                const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
                float psum = 0.0f;
                bf16x8 pb[2][2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        uint32_t w[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            w[e] = pack_bf16x2(__builtin_amdgcn_exp2f(st[kb][8 * u + 2 * e]),
                                               __builtin_amdgcn_exp2f(st[kb][8 * u + 2 * e + 1]));
                            psum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[e]), ones, psum,
                                                                   false);
                        }
                        pb[kb][u] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
                    }
                l_run += sum_halves(psum);

                // O^T += V^T P^T; chunk (kb, u): k index 8*hh + e <-> key 32*kb + 16*u + 8*(e/4) + 4*hh + (e%4)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int kr = 32 * kb + 16 * u + 4 * hh + tr_row;
#pragma unroll
                        for (int db = 0; db < 4; ++db) {
                            const uint16_t* base_v = &Vs[kr * kLdV + 32 * db + tr_col];
                            const shortx4 lo = lds_read_tr16(base_v);
                            const shortx4 hi = lds_read_tr16(base_v + 8 * kLdV);
                            const bf16x8 vf = __builtin_bit_cast(
                                bf16x8, (shortx8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
                            o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[kb][u], o[db], 0, 0, 0);
                        }
                    }
            }
            if (it + 1 < n_iter) stash(stage_base + ((it + 1) & 1) * kStage);
            __syncthreads();
        }

        // merge the two groups' partial results through LDS (the stage buffers are free now)
        float* xo = reinterpret_cast<float*>(smem) + wq * (64 * 64 + 3 * 64);
        if (grp == 1) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) xo[(16 * db + i) * 64 + lane] = o[db][i];
            xo[4096 + lane] = m_s;
            xo[4096 + 64 + lane] = m_t;
            xo[4096 + 128 + lane] = l_run;
        }
        __syncthreads();
        if (grp == 0) {
            const float m1s = xo[4096 + lane];
            const float m1t = xo[4096 + 64 + lane];
            const float l1 = xo[4096 + 128 + lane];
            const float ms = fmaxf(m_s, m1s);
            const float a0 = (m_s == kNegInf) ? 0.0f : exp2f(m_s - ms);
            const float a1 = (m1s == kNegInf) ? 0.0f : exp2f(m1s - ms);
            const float l = l_run * a0 + l1 * a1;
            const float mt = fmaxf(m_t, m1t);
            if (qrow < T) {
                const bool valid = qrow < L && l > 0.0f;
                const float inv = valid ? 1.0f / l : 0.0f;
                const float s0 = a0 * inv, s1 = a1 * inv;
                uint16_t* op = Og + (int64_t)qrow * a.ldo;
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int I = 0; I < 4; ++I) {
                        float v[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int i = 4 * I + r;
                            v[r] = o[db][i] * s0 + xo[(16 * db + i) * 64 + lane] * s1;
                        }
                        uint2 w;
                        w.x = pack_bf16x2(v[0], v[1]);
                        w.y = pack_bf16x2(v[2], v[3]);
                        *reinterpret_cast<uint2*>(&op[32 * db + 8 * I + 4 * hh]) = w;
                    }
                if (hh == 0) {
                    if (a.m) a.m[stat_base + (int64_t)qrow * a.H] = valid ? mt * (1.0f / kLog2e) : kNegInf;
                    if (a.l) a.l[stat_base + (int64_t)qrow * a.H] = valid ? l * exp2f(ms - mt) : 0.0f;
                }
            }
        }
        __syncthreads();
    }
}

int g_num_cus[64];

}  // namespace

int launch_flash_fwd_bf16(const FlashArgs& a, const SeqLens* lens, hipStream_t stream) {
    SeqLens sl;
    if (a.ragged) sl = *lens;
    else sl.len[0] = a.T;
    int dev = 0;
    DT_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return set_error(DT_ERR_UNSUPPORTED, "device index %d out of range", dev);
    if (g_num_cus[dev] == 0) {
        int n = 0;
        DT_HIP_TRY(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        g_num_cus[dev] = n > 0 ? n : 1;
    }
    if (a.ldk != a.ldv) return set_error(DT_ERR_UNSUPPORTED, "bf16 kernel needs equal K and V row strides");
    if ((int64_t)a.T * a.ldk * 2 >= ((int64_t)1 << 31))
        return set_error(DT_ERR_UNSUPPORTED, "K/V extent of one sequence exceeds 2 GiB");
    const int64_t n_items = (int64_t)((a.T + kBM - 1) / kBM) * a.B * a.H;
    if (n_items > 0x7fffffff) return set_error(DT_ERR_UNSUPPORTED, "too many attention items");
    const int grid = (int)(n_items < g_num_cus[dev] ? n_items : g_num_cus[dev]);
    hipLaunchKernelGGL(flash_fwd_bf16_kernel, dim3(grid), dim3(kThreads), 0, stream, a, sl);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
