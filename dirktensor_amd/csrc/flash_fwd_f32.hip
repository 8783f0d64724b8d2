// Causal flash attention forward, fp32 exact mode, for gfx950 (CDNA4).
//
// Replaces flash_attention_forward (FlashAttention.cpp:24-182). The reference
// runs 256x256 tiles with two cblas_sgemm calls per tile and a scalar softmax;
// here a persistent workgroup walks 128-query items (flash_items.h: snake order
// over items sorted by causal cost, so a long query tile is paired with a short
// one) and streams 32-key tiles of K and V through LDS. A launch that fits one
// round folds its units instead (flash_items.h): an item is then the 64-query
// tiles p and n-1-p of one (batch, head), rows 0-63 and 64-127.
//
// Work split: 8 waves in two groups of 4. Both groups hold the same 128 queries
// (32 per wave) and split the key tiles: group g takes tiles g, g+2, g+4, ... At
// the end group 1 hands its partial (max, sum, O) to group 0 through LDS and
// group 0 merges them with the same rescale the reference applies between tiles
// (FlashAttention.cpp:134-156). Each wave computes S^T = K Q^T for its 32
// queries with v_mfma_f32_32x32x2_f32, so that in the accumulator layout one
// lane holds one query (lane % 32) and 16 keys; the row max / row sum of the
// online softmax are then a per-lane reduction plus one exchange with lane ^ 32.
// The probabilities stay in the accumulator registers and feed the PV product
// O^T += V^T P^T directly as the B operand (the MFMA's k index is only a
// summation label, so V rows are read in the accumulator's key order).
//
// K and V tiles move from HBM straight into LDS with buffer_load ... lds,
// double-buffered: while a step computes on one stage, the group's next tile
// streams into the other; one barrier per step. Descriptors end at the
// sequence's last valid key, so rows past it arrive as zeros. LDS rows are 512
// bytes (128 floats), unpadded; the 16-byte chunk c of row r is stored at chunk
// position c ^ (r & 15), which keeps the row-wise K reads (16 rows, one chunk
// each) and the column-block V reads (one row, 16 chunks) free of bank conflicts.
//
// Numerics follow the reference: S = scale * Q K^T (FlashAttention.cpp:83-91),
// keys with k_pos > q_pos masked (:102), m = row max of the scaled scores,
// l = sum exp(s - m) (:159-163), output O / l, and a row with l == 0 written as
// zeros (:165-174). The online rescale uses the running max directly
// (FA-2 form) instead of the reference's tile-local max with alpha/beta
// factors (:134-156); both equal sum_k exp(s_k - m_final) up to rounding.
// exp is evaluated as exp2 with log2(e) folded into the scale.

#include "flash_items.h"

#include <type_traits>
#include <utility>

namespace dt {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kD = 128;                      // head_dim (model_config.h:3)
constexpr int kBM = kItemRows;               // queries per item
constexpr int kBN = 32;                      // keys per tile
constexpr int kThreads = 512;                // 8 waves
constexpr int kRowBytes = kD * 4;            // one K or V row, unpadded
constexpr int kTileBytes = kBN * kRowBytes;  // 16 KB per tensor per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr int kBufferDword3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

// one LDS stage: [group][K, V][tile bytes]
typedef uint8_t Stage[2][2][kTileBytes];

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
// calls f(std::integral_constant<int, I>{}) for I = 0 .. N-1 (compile-time unrolled)
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}
// keeps each group of MFMAs with the LDS read issued beside it: the scheduler may not move work across
#define DT_BUNDLE_END __builtin_amdgcn_sched_barrier(0)

// chunk position of 16-byte chunk c of an LDS row r
__device__ __forceinline__ int pos(int r, int c) { return c ^ (r & 15); }

// Buffer descriptor over [base, base + bytes): loads at or past the end return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferDword3);
}

// LDS DMA issued through inline assembly: the compiler does not track these loads, so it does not wait
// for them before reading the other LDS stage; stage_barrier() waits for them before any wave reads the
// stage they fill. M0 (an operand bound to M0) holds the wave-uniform LDS destination; lane i writes 16
// bytes at M0 + 16*i.
// The compiler cannot insert the wait states the hardware needs before these instructions (5 after a VALU
// write of an SGPR they read, such as a v_readlane reload of the descriptor; 1 after an SALU write of M0),
// since it does not see inside the asm: s_nop 4 provides them.
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_void*)p; }
__device__ __forceinline__ void dma16(uint32_t lds, uint32_t voff, __amdgpu_buffer_rsrc_t r) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds) : "memory");
}

// this wave's DMA and LDS accesses are complete before any wave passes
__device__ __forceinline__ void stage_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// LDS accesses only: vector memory requests in flight (output stores) are not waited for
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__global__ __launch_bounds__(kThreads, 1) void flash_fwd_f32_kernel(FlashArgs a, Schedule sc) {
    __shared__ __attribute__((aligned(1024))) Stage stage0;
    __shared__ __attribute__((aligned(1024))) Stage stage1;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;  // key-tile group
    // 32-query block within the item (also this wave's share of a DMA tile); in a folded launch group 1's
    // waves take the blocks in the other half, so each SIMD holds one wave of each 64-query tile
    const int wq = (wave & 3) ^ (sc.fold ? 2 * grp : 0);
    const int ln = lane & 31;   // query within the wave's 32 (MFMA n index)
    const int hh = lane >> 5;   // lane half (MFMA k index)

    // DMA: instruction n of wave wq fills LDS rows 2*(4n + wq) and 2*(4n + wq) + 1 of a tile (1 KB, 16 bytes
    // per lane at chunk position lane % 32); the lane fetches the global chunk that the swizzle puts there.
    uint32_t koff[4], voff[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        const int r = 2 * (4 * n + wq) + hh;
        const int c = pos(r, ln);  // pos is an involution: the chunk stored at position ln
        koff[n] = (uint32_t)((r * a.ldk + 4 * c) * 4);
        voff[n] = (uint32_t)((r * a.ldv + 4 * c) * 4);
    }

    const int T = a.T;
    const int G = gridDim.x;
    const float c = a.scale * kLog2e;

    for (int round = 0;; ++round) {
        const int k_unit = snake_item(round, G, (int)blockIdx.x);
        if (k_unit >= sc.n_units) break;
        const Unit u = decode_unit(k_unit, sc, a.H, sc.cum);  // a whole item: this kernel's schedules split nothing
        const int b = u.b, h = u.h;
        const int L = u.L;  // valid keys / rows of this sequence
        const int q0 = u.qa;
        const int qw0 = (wq < 2 ? u.qa : u.qb - 64) + wq * 32;  // first query of this wave
        const int qrow = qw0 + ln;

        const float* Qg = static_cast<const float*>(a.q) + (int64_t)b * T * a.ldq + (int64_t)h * kD;
        const float* Kg = static_cast<const float*>(a.k) + (int64_t)b * T * a.ldk + (int64_t)h * kD;
        const float* Vg = static_cast<const float*>(a.v) + (int64_t)b * T * a.ldv + (int64_t)h * kD;
        float* Og = static_cast<float*>(a.o) + (int64_t)b * T * a.ldo + (int64_t)h * kD;
        const int64_t stat_base = ((int64_t)b * T) * a.H + h;  // m/l index of row t: stat_base + t*H

        if (q0 >= L) {  // every row of this tile is padding: the reference's empty row (l == 0)
            if (grp == 0 && qrow < T) {
                const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
                for (int j = 0; j < 16; ++j) *reinterpret_cast<float4*>(&Og[(int64_t)qrow * a.ldo + 64 * hh + 4 * j]) = z;
                if (hh == 0) {
                    if (a.m) a.m[stat_base + (int64_t)qrow * a.H] = kNegInf;
                    if (a.l) a.l[stat_base + (int64_t)qrow * a.H] = 0.0f;
                }
            }
            continue;  // no LDS was touched: no barrier needed
        }

        const int k_end = a.causal ? min(u.qb + 64, L) : L;
        const int n_tiles = (k_end + kBN - 1) / kBN;
        const int n_steps = (n_tiles + 1) / 2;

        // K and V of tile kt of this group -> one LDS stage, straight from HBM
        auto dma = [&](Stage& stg, int kt) {
            const int k0 = kt * kBN;
            const __amdgpu_buffer_rsrc_t rk = make_rsrc(Kg + (int64_t)k0 * a.ldk, (uint32_t)(L - k0) * (uint32_t)a.ldk * 4u);
            const __amdgpu_buffer_rsrc_t rv = make_rsrc(Vg + (int64_t)k0 * a.ldv, (uint32_t)(L - k0) * (uint32_t)a.ldv * 4u);
            const uint32_t lk = __builtin_amdgcn_readfirstlane(lds_addr(&stg[grp][0][wq * 1024]));
            const uint32_t lv = __builtin_amdgcn_readfirstlane(lds_addr(&stg[grp][1][wq * 1024]));
#pragma unroll
            for (int n = 0; n < 4; ++n) dma16(lk + 4096 * n, koff[n], rk);
#pragma unroll
            for (int n = 0; n < 4; ++n) dma16(lv + 4096 * n, voff[n], rv);
        };
        // the first tile streams in while the query row loads
        if (grp < n_tiles) dma(stage0, grp);

        // Q fragment in registers: q[4*j + e] = Q[qrow][8*j + 4*hh + e] (B operand of S^T = K Q^T); all
        // sixteen loads are in flight before the first is used
        float q[64];
        {
            float4 raw[16];
            if (qrow < T) {
                const float* qp = Qg + (int64_t)qrow * a.ldq + 4 * hh;
#pragma unroll
                for (int j = 0; j < 16; ++j) raw[j] = *reinterpret_cast<const float4*>(qp + 8 * j);
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j) raw[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                q[4 * j + 0] = raw[j].x;
                q[4 * j + 1] = raw[j].y;
                q[4 * j + 2] = raw[j].z;
                q[4 * j + 3] = raw[j].w;
            }
        }

        // O^T accumulators: o[bb][i] holds O[q][d] with d = 4*m + bb, m = 8*(i/4) + 4*hh + (i%4).
        floatx16 o[4];
#pragma unroll
        for (int bb = 0; bb < 4; ++bb)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[bb][i] = 0.0f;
        float m_run = kNegInf;  // running max of the raw (unscaled) scores
        float l_run = 0.0f;

        // one 32-key tile of this wave's queries
        auto compute = [&](const Stage& stg, int k0) {
            const uint8_t* Ks = stg[grp][0];
            const uint8_t* Vs = stg[grp][1];
            // S^T: st[i] = S[qrow][key], key = k0 + 8*(i/4) + 4*hh + (i%4)
            floatx16 st;
#pragma unroll
            for (int i = 0; i < 16; ++i) st[i] = 0.0f;
            // K chunk j of row ln through a four-deep register ring, three reads ahead of its MFMAs
            auto read_k = [&](int j) {
                return *reinterpret_cast<const float4*>(Ks + ln * kRowBytes + (pos(ln, 2 * j + hh) << 4));
            };
            {
                float4 kr[4];
                kr[0] = read_k(0);
                kr[1] = read_k(1);
                kr[2] = read_k(2);
                static_for<16>([&](auto J) {
                    constexpr int j = decltype(J)::value;
                    if constexpr (j + 3 < 16) kr[(j + 3) & 3] = read_k(j + 3);
                    const float4 kv = kr[j & 3];
                    st = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, q[4 * j + 0], st, 0, 0, 0);
                    st = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, q[4 * j + 1], st, 0, 0, 0);
                    st = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, q[4 * j + 2], st, 0, 0, 0);
                    st = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, q[4 * j + 3], st, 0, 0, 0);
                    DT_BUNDLE_END;
                });
            }
            // mask (diagonal / ragged tail only) and tile max
            const bool need_mask = (a.causal && k0 + kBN - 1 > qw0) || (k0 + kBN > L);
            float tmax = kNegInf;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (need_mask) {
                    const int key = k0 + 8 * (i / 4) + 4 * hh + (i % 4);
                    if ((a.causal && key > qrow) || key >= L) st[i] = kNegInf;
                }
                tmax = fmaxf(tmax, st[i]);
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
                for (int i = 0; i < 16; ++i) {
                    const float p = __builtin_amdgcn_exp2f(st[i] * c - mc);
                    st[i] = p;
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
            // O^T += V^T P^T: MFMA step s takes key 8*(s/4) + 4*hh + (s%4) of the tile from lane half hh.
            auto read_v = [&](int s) {
                const int key = 8 * (s / 4) + 4 * hh + (s % 4);
                return *reinterpret_cast<const float4*>(Vs + key * kRowBytes + (pos(key, ln) << 4));
            };
            {
                float4 vr[4];
                vr[0] = read_v(0);
                vr[1] = read_v(1);
                vr[2] = read_v(2);
                static_for<16>([&](auto S) {
                    constexpr int s = decltype(S)::value;
                    if constexpr (s + 3 < 16) vr[(s + 3) & 3] = read_v(s + 3);
                    const float4 vv = vr[s & 3];
                    const float p = st[s];
                    o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, p, o[0], 0, 0, 0);
                    o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, p, o[1], 0, 0, 0);
                    o[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, p, o[2], 0, 0, 0);
                    o[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, p, o[3], 0, 0, 0);
                    DT_BUNDLE_END;
                });
            }
        };
        // compute from `cur` (tile kt) while the group's next tile kn streams into `nxt`
        auto step = [&](const Stage& cur, Stage& nxt, int kt, int kn) {
            if (kn < n_tiles) dma(nxt, kn);
            const int k0 = kt * kBN;
            if (kt >= n_tiles || (a.causal && k0 > qw0 + 31)) return;  // nothing of this tile is visible
            compute(cur, k0);
        };

        stage_barrier();  // the first tile has landed
        for (int it = 0; it < n_steps; it += 2) {
            step(stage0, stage1, 2 * it + grp, 2 * (it + 1) + grp);
            stage_barrier();
            if (it + 1 >= n_steps) break;
            step(stage1, stage0, 2 * (it + 1) + grp, 2 * (it + 2) + grp);
            stage_barrier();
        }

        // group 1 hands (O, m, l) to group 0 through LDS (no DMA is in flight now): O as 16 float4 per lane
        float4* xo = reinterpret_cast<float4*>(&stage0[0][0][0]) + wq * (16 * 64);
        float* xs = reinterpret_cast<float*>(&stage1[0][0][0]) + wq * (2 * 64);
        if (grp == 1) {
#pragma unroll
            for (int i = 0; i < 16; ++i) xo[i * 64 + lane] = make_float4(o[0][i], o[1][i], o[2][i], o[3][i]);
            xs[lane] = m_run;
            xs[64 + lane] = l_run;
        }
        lds_barrier();
        if (grp == 0) {
            // finalize (FlashAttention.cpp:159-175) over both groups' keys
            const float m1 = xs[lane];
            const float l1 = xs[64 + lane];
            const float m = fmaxf(m_run, m1);
            const float m_use = (m == kNegInf) ? 0.0f : m;
            const float a0 = exp2f((m_run - m_use) * c);  // 0 for a group that saw no valid key
            const float a1 = exp2f((m1 - m_use) * c);
            const float l = l_run * a0 + l1 * a1;
            if (qrow < T) {
                const bool valid = qrow < L && l > 0.0f;
                float* op = Og + (int64_t)qrow * a.ldo;
#pragma unroll
                for (int I = 0; I < 4; ++I)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = 4 * I + r;
                        const float4 x = xo[i * 64 + lane];
                        float4 v;
                        if (valid) {
                            v.x = (o[0][i] * a0 + x.x * a1) / l;
                            v.y = (o[1][i] * a0 + x.y * a1) / l;
                            v.z = (o[2][i] * a0 + x.z * a1) / l;
                            v.w = (o[3][i] * a0 + x.w * a1) / l;
                        } else {
                            v = make_float4(0.f, 0.f, 0.f, 0.f);
                        }
                        *reinterpret_cast<float4*>(&op[32 * I + 16 * hh + 4 * r]) = v;
                    }
                if (hh == 0) {
                    if (a.m) a.m[stat_base + (int64_t)qrow * a.H] = valid ? m * a.scale : kNegInf;
                    if (a.l) a.l[stat_base + (int64_t)qrow * a.H] = valid ? l : 0.0f;
                }
            }
        }
        // group 0 has read the exchange before the next item's DMA may overwrite it; the output stores
        // need not have completed
        lds_barrier();
    }
}

}  // namespace

int launch_flash_fwd_f32(const FlashArgs& a, const SeqLens* lens, hipStream_t stream) {
    SeqLens sl;
    if (a.ragged) sl = *lens;
    else sl.len[0] = a.T;
    const int64_t ld = a.ldk > a.ldv ? a.ldk : a.ldv;
    if ((int64_t)a.T * ld * 4 >= ((int64_t)1 << 31))
        return set_error(DT_ERR_UNSUPPORTED, "K/V extent of one sequence exceeds 2 GiB");
    int grid = 0;
    DT_TRY(persistent_grid((int64_t)((a.T + kBM - 1) / kBM) * a.B * a.H, &grid));
    Schedule sc;
    build_schedule(a, sl, grid, false, &sc, true);
    hipLaunchKernelGGL(flash_fwd_f32_kernel, dim3(grid), dim3(kThreads), 0, stream, a, sc);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
