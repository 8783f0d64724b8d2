// Causal flash attention forward, bf16 MFMA mode, for gfx950 (CDNA4).
//
// Replaces flash_attention_forward (FlashAttention.cpp:24-182) with bf16
// Q/K/V/O, fp32 accumulation and an fp32 online softmax.
//
// Work decomposition
//   * An item is 128 queries of one (batch, head). A persistent grid of at most
//     one workgroup per CU walks a list of work units (flash_items.h) in "snake"
//     order over decreasing causal cost, so a workgroup pairs a long query tile
//     with a short one; at T = 4096, H = 16 every workgroup gets 33 key tiles of
//     work. When the largest item costs at least twice a workgroup's fair share
//     (few heads, e.g. a tensor-parallel shard), items are split into parts of
//     consecutive key tiles on different workgroups; each part writes its
//     partial (m, l, O) to a workspace and the last one to finish merges them.
//   * A launch that fits one round folds its units (flash_items.h): a unit is then
//     the 64-query tiles p and n-1-p of one (batch, head), as one 128-query item
//     whose rows 0-63 are tile p, so every workgroup gets the same work.
//   * A workgroup has 8 waves in two groups of 4. Both groups hold the same 128
//     queries (32 per wave) and split the key tiles: group g takes 64-key tiles
//     g, g+2, g+4, ... At the end group 1 hands its partial (max, sum, O) to
//     group 0 through LDS and group 0 merges them with the same rescale the
//     reference applies between tiles (FlashAttention.cpp:134-156).
//   * K and V tiles move from HBM straight into LDS with buffer_load ... lds
//     (no staging registers), double-buffered in two LDS arrays: while a step
//     computes on one array, the next tile streams into the other (its K rows
//     after the step's S chain, its V rows after the softmax, so no DMA write
//     lands while this step's K fragments are read); one barrier per step.
//     The descriptors end at the sequence's last valid key, so rows
//     past it arrive as zeros. LDS rows are 256 bytes, unpadded; the 16-byte
//     chunk c of row r is stored at chunk position c ^ f(r),
//     f(r) = 4*(r & 3) + ((r >> 2) & 3), which keeps both the row-wise K reads
//     and the transposing V reads free of bank conflicts.
//   * Within a wave, S^T = K Q^T comes from v_mfma_f32_32x32x16_bf16 with K
//     rows from LDS as the A operand and the wave's Q fragment, held in
//     registers, as B; one lane then owns one query and 16 keys per 32-key
//     block, so the row max and row sum are a per-lane reduction plus one
//     exchange between the lane halves. P is converted to bf16 in registers
//     and used as the B operand of O^T += V^T P^T; the A operand (V^T) comes
//     from the gfx950 transposing LDS read ds_read_b64_tr_b16, where a 16-lane
//     group reads a 4-key x 16-dim block and each lane receives one dim column
//     of 4 keys, i.e. the MFMA's 8-key k slice taken as two 4-key runs in the
//     accumulator's key order.
//   * Both products read their LDS fragments through four-deep register rings,
//     three reads ahead of the MFMA that consumes them, so no MFMA waits for a
//     read issued just before it.
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
// The two lane halves that share a query keep their own m_t and l (over their
// own keys) and exchange them only when m_s must move and once at the end, so
// the common path of a tile has no cross-lane traffic; m_s itself is always
// the same in both halves.
// Keys with k_pos > q_pos are masked (FlashAttention.cpp:102); a row with no
// valid key is written as the reference's empty row (FlashAttention.cpp:165-174).

#include "flash_items.h"

#include <algorithm>
#include <atomic>
#include <type_traits>
#include <utility>

namespace dt {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef short shortx8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;
typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned v4u32 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kBN = 64;        // keys per tile
constexpr int kThreads = 512;  // 8 waves
constexpr int kRowBytes = 256;               // one K or V row (128 bf16), unpadded
constexpr int kTileBytes = kBN * kRowBytes;  // 16 KB per tensor per tile
constexpr int kObufRow = kRowBytes + 16;     // a row of the output staging tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kRescaleLog2 = 8.0f;
constexpr int kBufferDword3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

// one LDS stage: [group][K, V][tile bytes]
typedef uint8_t Stage[2][2][kTileBytes];

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 r = __builtin_convertvector((floatx2){lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, r);
}

// Row reductions over the two lane halves (lane l and lane l ^ 32 hold the same query), through
// v_permlane32_swap (VALU, no LDS crossbar) with x as both operands: the result pair holds, in every lane, the
// lower half's value and the upper half's (same order in both halves).
__device__ __forceinline__ float max_halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ shortx4 lds_read_tr16(const uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(p));
}

// Buffer descriptor over [base, base + bytes): loads at or past the end return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferDword3);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// chunk swizzle of an LDS row: chunk c of row r lives at position c ^ swz(r)
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// Per-wave state of one item.
struct Acc {
    floatx16 o[4];    // O^T: o[db][i] = O[qrow][32*db + 8*(i/4) + 4*hh + (i%4)] (unnormalised)
    floatx16 neg_ms;  // -m_s (0 while m_s is -inf), the starting accumulator of the S chain
    float m_t, m_s, l;
};

template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
// calls f(std::integral_constant<int, I>{}) for I = 0 .. N-1 (compile-time unrolled)
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}
// keeps each MFMA with the LDS read issued beside it: the scheduler may not move work across
#define DT_BUNDLE_END __builtin_amdgcn_sched_barrier(0)

// LDS fragment reads of one 64-key tile.
// K fragment r = 2*cc + kb: rows 32*kb + ln, dims 16*cc + 8*hh .. +8 (kaddr[cc]: block kb = 0).
__device__ __forceinline__ bf16x8 read_k(const uint8_t* Ks, const uint32_t (&kaddr)[8], int r) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(Ks + kaddr[r >> 1] + (r & 1) * 8192));
}
// V^T chunk c = 8*kb + 4*u + db: keys 32*kb + 16*u .. +16 (two transposing reads), dims 32*db .. +32.
// vaddr[s][db]: this lane's read s of dim block db in 16-key chunk 0; chunk (kb, u) adds 8192*kb + 4096*u.
__device__ __forceinline__ bf16x8 read_v(const uint8_t* Vs, const uint32_t (&vaddr)[2][4], int c) {
    const int rows = (c >> 3) * 8192 + ((c >> 2) & 1) * 4096;
    const int db = c & 3;
    const shortx4 lo = lds_read_tr16(Vs + vaddr[0][db] + rows);
    const shortx4 hi = lds_read_tr16(Vs + vaddr[1][db] + rows + 2048);
    return __builtin_bit_cast(bf16x8, (shortx8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
}

// One 64-key tile for one wave: S^T, softmax update, O^T += V^T P^T. Both products read their LDS
// fragments through four-deep rings, three reads ahead of the MFMA that consumes them, so an MFMA never
// waits for a read issued just before it.
// mid(0) runs after the S chain and mid(1) between the softmax and the PV product (the caller issues the
// next tile's K and V DMA there).
template <typename Mid>
__device__ __forceinline__ void tile_step(Acc& A, const bf16x8 (&qf)[8], const uint8_t* Ks, const uint8_t* Vs,
                                          const uint32_t (&kaddr)[8], const uint32_t (&vaddr)[2][4], int k0,
                                          bool need_mask, int lim, int hh, Mid&& mid) {
    floatx16 st[2];
    {
        bf16x8 kr[4];
        kr[0] = read_k(Ks, kaddr, 0);
        kr[1] = read_k(Ks, kaddr, 1);
        kr[2] = read_k(Ks, kaddr, 2);
        static_for<16>([&](auto R) {
            constexpr int r = decltype(R)::value;  // = 2*cc + kb
            if constexpr (r + 3 < 16) kr[(r + 3) & 3] = read_k(Ks, kaddr, r + 3);
            st[r & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kr[r & 3], qf[r >> 1], (r >> 1) == 0 ? A.neg_ms : st[r & 1],
                                                                0, 0, 0);
            DT_BUNDLE_END;
        });
    }
    mid(0);
    // the first V chunks stream in while the softmax runs
    bf16x8 vr[4];
    vr[0] = read_v(Vs, vaddr, 0);
    vr[1] = read_v(Vs, vaddr, 1);
    vr[2] = read_v(Vs, vaddr, 2);

    if (need_mask) {  // diagonal / ragged-tail tiles: selects, no per-element branches
        asm volatile("");  // keeps this rare block a branch (it must not be speculated into every tile)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = k0 + 32 * kb + 8 * (i / 4) + 4 * hh + (i % 4);
                st[kb][i] = key > lim ? kNegInf : st[kb][i];
            }
    }
    float tm0 = kNegInf, tm1 = kNegInf;  // two independent chains
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        tm0 = fmaxf(tm0, st[0][i]);
        tm1 = fmaxf(tm1, st[1][i]);
    }
    const float tmax = fmaxf(tm0, tm1);  // this lane half's maximum of t
    const float base = (A.m_s == kNegInf) ? 0.0f : A.m_s;  // what the S chain subtracted
    A.m_t = fmaxf(A.m_t, tmax + base);                      // this half's running maximum
    const bool grow = (A.m_s == kNegInf) ? (tmax > kNegInf) : (tmax > kRescaleLog2);
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // wave-uniform, rare after the first tile
        asm volatile("");  // keeps this rare block a branch (it must not be speculated into every tile)
        const float m_new = max_halves(A.m_t);     // the query's maximum over both halves
        const float delta = (m_new == kNegInf) ? 0.0f : m_new - base;
        const float alpha = (A.m_s == kNegInf) ? 0.0f : exp2f(A.m_s - m_new);
        A.m_s = m_new;
        A.l *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) A.o[db][i] *= alpha;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) st[kb][i] -= delta;
        const float nm = (A.m_s == kNegInf) ? 0.0f : -A.m_s;
#pragma unroll
        for (int i = 0; i < 16; ++i) A.neg_ms[i] = nm;
    }
    // p = exp2(t) in bf16; the row sum is over the bf16 values the PV product uses
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
    float psum[2] = {0.0f, 0.0f};
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
                psum[kb] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[e]), ones, psum[kb], false);
            }
            pb[kb][u] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
        }
    A.l += psum[0] + psum[1];  // this half's keys only
    mid(1);

    // O^T += V^T P^T; chunk (kb, u): k index 8*hh + e <-> key 32*kb + 16*u + 8*(e/4) + 4*hh + (e%4)
    static_for<16>([&](auto C) {
        constexpr int c = decltype(C)::value;  // = 8*kb + 4*u + db
        if constexpr (c + 3 < 16) vr[(c + 3) & 3] = read_v(Vs, vaddr, c + 3);
        A.o[c & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vr[c & 3], pb[c >> 3][(c >> 2) & 1], A.o[c & 3], 0, 0, 0);
        DT_BUNDLE_END;
    });
}

// 16 bytes to / from a buffer with device-scope coherence (cache policy sc1): the access goes through to
// the memory all XCDs share instead of stopping in this XCD's L2.
constexpr int kCoherent = 16;  // sc1
__device__ __forceinline__ void store_coherent(float4 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32, v), r, off, 0, kCoherent);
}
__device__ __forceinline__ float4 load_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCoherent));
}

// Barrier for the double-buffered loop: this wave's LDS DMA and LDS accesses are
// complete before any wave passes it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// Barrier over LDS accesses only: vector memory requests in flight are not waited for.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__global__ __launch_bounds__(kThreads, 1) void flash_fwd_bf16_kernel(FlashArgs a, Schedule sc) {
    __shared__ __attribute__((aligned(1024))) Stage stage0;
    __shared__ __attribute__((aligned(1024))) Stage stage1;
    __shared__ int last_part;  // this workgroup completes a split item
    __shared__ int cum_lds[kMaxKinds + 1];  // the schedule's unit counts (searched once per unit)

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, held in an SGPR
    const int grp = wave >> 2;  // key-tile group
    // 32-query block within the item (also this wave's share of a DMA tile). In a folded launch group 1's
    // waves take the blocks in the other half, so each SIMD (waves w and w + 4) holds one wave of each
    // 64-query tile and keeps one wave busy after the lower tile's keys run out.
    const int wq = (wave & 3) ^ (sc.fold ? 2 * grp : 0);
    const int ln = lane & 31;
    const int hh = lane >> 5;

    // DMA: instruction i of wave wq fills rows 16*i + 4*wq + lane/16 of a tile, 16 bytes per lane at
    // chunk position lane%16; the lane fetches the global chunk that the swizzle puts there.
    uint32_t voff[4];
    {
        const int rlo = lane >> 4;
        const int chunk = (lane & 15) ^ (4 * rlo + wq);  // swz(16*i + 4*wq + rlo) does not depend on i
#pragma unroll
        for (int i = 0; i < 4; ++i) voff[i] = (uint32_t)(((16 * i + 4 * wq + rlo) * a.ldk + 8 * chunk) * 2);
    }
    // Q DMA of an item's 128 rows: instruction i of wave w fills rows 32*i + 4*w + lane/16, in the same
    // swizzled layout (swz(32*i + 4*w + lane/16) = 4*(lane/16) + (w & 3) does not depend on i); instructions
    // 0-1 read the item's first 64 rows and 2-3 its second 64, each from its own base
    uint32_t qoff[2];
    {
        const int rlo = lane >> 4;
        const int chunk = (lane & 15) ^ (4 * rlo + (wave & 3));
#pragma unroll
        for (int i = 0; i < 2; ++i) qoff[i] = (uint32_t)(((32 * i + 4 * wave + rlo) * a.ldq + 8 * chunk) * 2);
    }
    // K fragment reads: row 32*kb + ln, chunk 2*cc + hh
    uint32_t kaddr[8];
    {
        const int g = hh ^ swz(ln);
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) kaddr[cc] = (uint32_t)(ln * kRowBytes + (((2 * cc) ^ g) << 4));
    }
    // V transposing reads: lane i of 16-lane group G reads row 4*hh + i/4 (+8 for the second read)
    // of a 16-key chunk, dims 32*db + 16*(G&1) + 4*(i&3) .. +3
    uint32_t vaddr[2][4];
    {
        const int i16 = lane & 15;
        const int tr_row = i16 >> 2;
        const int g2 = (lane >> 4) & 1;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int r = 4 * hh + tr_row + 8 * s;
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const int chunk = 4 * db + 2 * g2 + ((i16 & 3) >> 1);
                vaddr[s][db] = (uint32_t)((r - 8 * s) * kRowBytes + ((chunk ^ swz(r)) << 4) + 8 * (i16 & 1));
            }
        }
    }

    const int T = a.T;
    const int G = gridDim.x;
    const float c = a.scale * kLog2e;

    // a unit is decoded one round ahead (a search of the kind table, a chain of scalar loads), while the
    // previous unit's first tile is on its way
    if (!sc.dense) {
        for (int j = tid; j <= sc.n_kinds; j += kThreads) cum_lds[j] = sc.cum[j];
        __syncthreads();
    }
    int k_unit = snake_item(0, G, (int)blockIdx.x);
    Unit u_next = decode_unit(k_unit < sc.n_units ? k_unit : 0, sc, a.H, cum_lds);
    for (int round = 0; k_unit < sc.n_units; ++round) {
        const Unit u = u_next;
        const int k_next = snake_item(round + 1, G, (int)blockIdx.x);
        const int b = u.b, h = u.h;
        const int L = u.L;
        const int q0 = u.qa;
        const int qw0 = (wq < 2 ? u.qa : u.qb - 64) + wq * 32;  // this wave's first query
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
            k_unit = k_next;
            if (k_next < sc.n_units) u_next = decode_unit(k_next, sc, a.H, cum_lds);
            continue;  // no LDS was touched: no barrier needed
        }

        const int k_end = a.causal ? min(u.qb + 64, L) : L;
        // this unit's key tiles t0 .. t1-1: the whole item, or part u.part of S tiles (the last one the rest)
        const int n_item_tiles = (k_end + kBN - 1) / kBN;
        const int t0 = u.parts > 1 ? u.part * sc.S : 0;
        const int t1 = u.parts > 1 ? min(t0 + sc.S, n_item_tiles) : n_item_tiles;
        const int n_iter = max(t1 - t0 + 1, 0) / 2;

        // K (kv = 0) or V (kv = 1) of tile kt of this group -> one LDS stage, straight from HBM
        auto dma = [&](Stage& stg, int kv, int kt) {
            const int k0 = kt * kBN;
            const uint32_t bytes = (uint32_t)(L - k0) * (uint32_t)a.ldk * 2u;  // rows k0 .. L-1
            const __amdgpu_buffer_rsrc_t r = make_rsrc((kv ? Vg : Kg) + (int64_t)k0 * a.ldk, bytes);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)&stg[grp][kv][(4 * i + wq) * 1024], 16, voff[i],
                                                         0, 0, 0);
        };
        // The first tile streams into stage0 and the item's 128 query rows into stage1 (free until step 0),
        // both as whole 256-byte rows; rows past T arrive as zeros.
        if (t0 + grp < t1) {
            dma(stage0, 0, t0 + grp);
            dma(stage0, 1, t0 + grp);
        }
        uint8_t* Qs = &stage1[0][0][0];  // 128 rows x 256 bytes (group 0's K and V areas of stage1)
        {
            const __amdgpu_buffer_rsrc_t rqa = make_rsrc(Qg + (int64_t)u.qa * a.ldq, (uint32_t)(T - u.qa) * (uint32_t)a.ldq * 2u);
            const __amdgpu_buffer_rsrc_t rqb =
                make_rsrc(Qg + (int64_t)u.qb * a.ldq, (uint32_t)max(T - u.qb, 0) * (uint32_t)a.ldq * 2u);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rqa, (lds_void*)(Qs + wave * 1024), 16, qoff[0], 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rqa, (lds_void*)(Qs + 8192 + wave * 1024), 16, qoff[1], 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rqb, (lds_void*)(Qs + 16384 + wave * 1024), 16, qoff[0], 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rqb, (lds_void*)(Qs + 24576 + wave * 1024), 16, qoff[1], 0, 0, 0);
        }
        if (k_next < sc.n_units) u_next = decode_unit(k_next, sc, a.H, cum_lds);

        bf16x8 qf[8];  // filled from the Q tile once it has landed
        Acc A;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) A.o[db][i] = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) A.neg_ms[i] = 0.0f;
        A.m_t = kNegInf;
        A.m_s = kNegInf;
        A.l = 0.0f;

        // Step on stage `cur` (tile kt) while the group's next tile kn streams into `nxt`: its K after the
        // step's S chain, its V after the softmax, so no DMA write lands in LDS while this step's K fragments
        // are read (K at the start of the step, or K and V both there, measured 1.3-3 % slower).
        auto step = [&](const Stage& cur, Stage& nxt, int kt, int kn) {
            const bool dn = kn < t1;
            auto mid = [&](int kv) {  // 0: K, 1: V
                if (dn) dma(nxt, kv, kn);
            };
            const int k0 = kt * kBN;
            if (kt >= t1 || (a.causal && k0 > qw0 + 31)) {  // nothing of this tile is visible
                mid(0);
                mid(1);
                return;
            }
            const bool need_mask = (a.causal && k0 + kBN - 1 > qw0) || k0 + kBN > L;
            const int lim = a.causal ? min(qrow, L - 1) : L - 1;  // keys > lim are masked
            tile_step(A, qf, cur[grp][0], cur[grp][1], kaddr, vaddr, k0, need_mask, lim, hh, mid);
        };

        stage_barrier();  // the first tile and the query rows have landed
        // Q fragment, pre-multiplied by scale * log2 e: qf[cc] = Q[qrow][16*cc + 8*hh .. +8] * c
        // (row 32*wq + ln of the Q tile, read like a K fragment)
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) {
            const uint4 raw = *reinterpret_cast<const uint4*>(Qs + wq * 8192 + kaddr[cc]);
            const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
            uint32_t sw[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) sw[e] = pack_bf16x2(bf16_lo(w[e]) * c, bf16_hi(w[e]) * c);
            qf[cc] = __builtin_bit_cast(bf16x8, make_uint4(sw[0], sw[1], sw[2], sw[3]));
        }
        lds_barrier();  // every wave holds its Q fragment before step 0's DMA refills stage1
        for (int it = 0; it < n_iter; it += 2) {
            // even step: compute from stage0 while the group's next tile streams into stage1
            step(stage0, stage1, t0 + 2 * it + grp, t0 + 2 * (it + 1) + grp);
            stage_barrier();
            if (it + 1 >= n_iter) break;
            // odd step: compute from stage1 while the tile after it streams into stage0
            step(stage1, stage0, t0 + 2 * (it + 1) + grp, t0 + 2 * (it + 2) + grp);
            stage_barrier();
        }

        // combine the lane halves' maxima and sums, then merge the two groups through LDS: group g finalises
        // dims 64g .. 64g+63 (dim blocks 2g, 2g+1) of its block's rows and hands the other half of its partial
        // O to the other group (no DMA is in flight now)
        A.m_t = max_halves(A.m_t);
        A.l = sum_halves(A.l);
        // group g's handed-over half of block wq: float4 k = 4*(db - 2*(1-g)) + I of lane `lane` at
        // xo(g)[k*64 + lane] (8 KB per wave and group, stage0); its (m_s, m_t, l) at xs(g) (stage1)
        auto xo = [&](int g) { return reinterpret_cast<float4*>(&stage0[0][0][0]) + (g * 4 + wq) * (8 * 64); };
        auto xs = [&](int g) { return reinterpret_cast<float*>(&stage1[0][0][0]) + (g * 4 + wq) * (3 * 64); };
        uint8_t* obuf = &stage1[0][0][0] + 8192;  // the output tile on its way to HBM (128 x 272 bytes, after xs)
        {
            float4* out = xo(grp);
            auto hand = [&](auto DB) {
                constexpr int db = decltype(DB)::value;
#pragma unroll
                for (int I = 0; I < 4; ++I)
                    out[(4 * (db & 1) + I) * 64 + lane] = make_float4(A.o[db][4 * I], A.o[db][4 * I + 1], A.o[db][4 * I + 2], A.o[db][4 * I + 3]);
            };
            if (grp == 0) {
                hand(std::integral_constant<int, 2>{});
                hand(std::integral_constant<int, 3>{});
            } else {
                hand(std::integral_constant<int, 0>{});
                hand(std::integral_constant<int, 1>{});
            }
            float* st = xs(grp);
            st[lane] = A.m_s;
            st[64 + lane] = A.m_t;
            st[128 + lane] = A.l;
        }
        __syncthreads();
        // part p's partial result in the workspace (split items), and a float4's byte offset in it
        auto partial_rsrc = [&](int part) {
            return make_rsrc(a.split_ws + ((size_t)u.slot * kMaxParts + part) * kPartialFloats, (uint32_t)(kPartialFloats * 4));
        };
        auto pslot = [&](int k) { return (uint32_t)(((wq * 17 + k) * 64 + lane) * 16); };
        {
            // both groups form the same statistics, group 0's terms first
            const float* so = xs(1 - grp);
            const float os = so[lane], ot = so[64 + lane], ol = so[128 + lane];
            const float m0s = grp ? os : A.m_s, m1s = grp ? A.m_s : os;
            const float m0t = grp ? ot : A.m_t, m1t = grp ? A.m_t : ot;
            const float l0 = grp ? ol : A.l, l1 = grp ? A.l : ol;
            const float ms = fmaxf(m0s, m1s);
            const float a0 = (m0s == kNegInf) ? 0.0f : exp2f(m0s - ms);
            const float a1 = (m1s == kNegInf) ? 0.0f : exp2f(m1s - ms);
            const float l = l0 * a0 + l1 * a1;
            const float mt = fmaxf(m0t, m1t);
            const float4* in = xo(1 - grp);
            // v = O0 * c0 + O1 * c1 over dim block db (this group's): its own O and the other group's half
            auto merged = [&](auto DB, int I, float c0, float c1, float (&v)[4]) {
                constexpr int db = decltype(DB)::value;
                const float4 x = in[(4 * (db & 1) + I) * 64 + lane];
                const float xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float own = A.o[db][4 * I + r];
                    v[r] = (db < 2) ? own * c0 + xv[r] * c1 : xv[r] * c0 + own * c1;
                }
            };
            if (u.parts == 1) {
                // the output rows go to LDS (row-major, rows padded to 272 bytes so the 32 rows a write
                // instruction touches fall in different banks) and from there to HBM as whole rows, below
                const bool valid = qrow < L && l > 0.0f;
                const float inv = valid ? 1.0f / l : 0.0f;
                const float s0 = a0 * inv, s1 = a1 * inv;
                const int orow = 32 * wq + ln;
                auto fin = [&](auto DB) {
                    constexpr int db = decltype(DB)::value;
#pragma unroll
                    for (int I = 0; I < 4; ++I) {
                        float v[4];
                        merged(DB, I, s0, s1, v);
                        uint2 w;
                        w.x = pack_bf16x2(v[0], v[1]);
                        w.y = pack_bf16x2(v[2], v[3]);
                        *reinterpret_cast<uint2*>(obuf + orow * kObufRow + 16 * (4 * db + I) + 8 * hh) = w;
                    }
                };
                if (grp == 0) {
                    fin(std::integral_constant<int, 0>{});
                    fin(std::integral_constant<int, 1>{});
                    if (qrow < T && hh == 0) {
                        if (a.m) a.m[stat_base + (int64_t)qrow * a.H] = valid ? mt * (1.0f / kLog2e) : kNegInf;
                        if (a.l) a.l[stat_base + (int64_t)qrow * a.H] = valid ? l * exp2f(ms - mt) : 0.0f;
                    }
                } else {
                    fin(std::integral_constant<int, 2>{});
                    fin(std::integral_constant<int, 3>{});
                }
            } else {
                // this part's O relative to ms, both groups' keys, and (m_s, m_t, l) -> its workspace slot in
                // register order: float4 k = 4*db + I of lane `lane` of wave wq at ((wq*17 + k)*64 + lane)*16
                // bytes, k = 16 the statistics (1 KB contiguous per store instruction); each group its dims
                const __amdgpu_buffer_rsrc_t rp = partial_rsrc(u.part);
                auto put = [&](auto DB) {
                    constexpr int db = decltype(DB)::value;
#pragma unroll
                    for (int I = 0; I < 4; ++I) {
                        float v[4];
                        merged(DB, I, a0, a1, v);
                        store_coherent(make_float4(v[0], v[1], v[2], v[3]), rp, pslot(4 * db + I));
                    }
                };
                if (grp == 0) {
                    put(std::integral_constant<int, 0>{});
                    put(std::integral_constant<int, 1>{});
                    store_coherent(make_float4(ms, mt, l, 0.0f), rp, pslot(16));
                } else {
                    put(std::integral_constant<int, 2>{});
                    put(std::integral_constant<int, 3>{});
                }
            }
        }
        if (u.parts == 1) {  // the item's 128 output rows: 16 lanes per 256-byte row, 4 rows per store instruction
            lds_barrier();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int ch = j * kThreads + tid;  // 16-byte chunk ch % 16 of row ch / 16
                const int r = ch >> 4, c = ch & 15;
                const int qr = (j < 2 ? u.qa : u.qb - 64) + r;  // rows 0-63 in j = 0, 1; rows 64-127 in j = 2, 3
                const uint4 w = *reinterpret_cast<const uint4*>(obuf + r * kObufRow + 16 * c);
                // streaming (non-temporal) stores: whole 256-byte rows this kernel never reads back
                if (qr < T)
                    __builtin_nontemporal_store((u32x4){w.x, w.y, w.z, w.w},
                                                reinterpret_cast<u32x4*>(&Og[(int64_t)qr * a.ldo + 8 * c]));
            }
        }
        if (u.parts > 1) {  // the same for every wave of the workgroup
            // The last of the item's parts to arrive merges them all, in part order, from the workspace; the
            // counter goes back to zero for the next launch. The partials are written and read with device-scope
            // coherent accesses (sc1: through to, and from, the memory every XCD sees), so no L2 write-back or
            // invalidate is needed: a partial is complete once its stores are (vmcnt), before it is counted.
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (tid == 0) {
                const int prev = __hip_atomic_fetch_add(&a.split_cnt[u.slot], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int last = prev == u.parts - 1;
                if (last) __hip_atomic_store(&a.split_cnt[u.slot], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                last_part = last;
            }
            __syncthreads();
            if (last_part) {
                // group g merges dims 64g .. 64g+63 (float4 k = 8g .. 8g+7). The statistics of every part and the
                // O values of parts 0 and 1 are requested together (a third part's after them)
                float4 st[kMaxParts], x[2][8];
#pragma unroll
                for (int p = 0; p < kMaxParts; ++p)
                    if (p < u.parts) st[p] = load_coherent(partial_rsrc(p), pslot(16));
#pragma unroll
                for (int p = 0; p < 2; ++p)
#pragma unroll
                    for (int j = 0; j < 8; ++j) x[p][j] = load_coherent(partial_rsrc(p), pslot(8 * grp + j));
                float ms = kNegInf, mt = kNegInf;
#pragma unroll
                for (int p = 0; p < kMaxParts; ++p)
                    if (p < u.parts) {
                        ms = fmaxf(ms, st[p].x);
                        mt = fmaxf(mt, st[p].y);
                    }
                float l = 0.0f;
                float4 acc[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                auto accumulate = [&](int p, const float4 (&xp)[8]) {  // in part order
                    const float ap = (st[p].x == kNegInf) ? 0.0f : exp2f(st[p].x - ms);
                    l += st[p].z * ap;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        acc[j].x += xp[j].x * ap;
                        acc[j].y += xp[j].y * ap;
                        acc[j].z += xp[j].z * ap;
                        acc[j].w += xp[j].w * ap;
                    }
                };
                accumulate(0, x[0]);
                accumulate(1, x[1]);
                if (u.parts > 2) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) x[0][j] = load_coherent(partial_rsrc(2), pslot(8 * grp + j));
                    accumulate(2, x[0]);
                }
                if (qrow < T) {
                    const bool valid = qrow < L && l > 0.0f;
                    const float inv = valid ? 1.0f / l : 0.0f;
                    uint16_t* op = Og + (int64_t)qrow * a.ldo;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {  // k = 8*grp + j = 4*db + I
                        const int k = 8 * grp + j;
                        uint2 w;
                        w.x = pack_bf16x2(acc[j].x * inv, acc[j].y * inv);
                        w.y = pack_bf16x2(acc[j].z * inv, acc[j].w * inv);
                        *reinterpret_cast<uint2*>(&op[32 * (k >> 2) + 8 * (k & 3) + 4 * hh]) = w;
                    }
                    if (grp == 0 && hh == 0) {
                        if (a.m) a.m[stat_base + (int64_t)qrow * a.H] = valid ? mt * (1.0f / kLog2e) : kNegInf;
                        if (a.l) a.l[stat_base + (int64_t)qrow * a.H] = valid ? l * exp2f(ms - mt) : 0.0f;
                    }
                }
            }
        }
        // group 0 has read the exchange (its LDS reads are complete) before the next item's DMA may overwrite
        // it; the output stores need not have completed
        lds_barrier();
        k_unit = k_next;
    }
}

}  // namespace

int persistent_grid(int64_t n_items, int* grid) {
    static std::atomic<int> num_cus[64];  // per device, filled on first use (any thread; same value)
    int dev = 0;
    DT_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return set_error(DT_ERR_UNSUPPORTED, "device index %d out of range", dev);
    int cus = num_cus[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
        int n = 0;
        DT_HIP_TRY(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        cus = n > 0 ? n : 1;
        num_cus[dev].store(cus, std::memory_order_relaxed);
    }
    if (n_items > 0x7fffffff) return set_error(DT_ERR_UNSUPPORTED, "too many attention items");
    *grid = (int)(n_items < cus ? n_items : cus);
    return DT_OK;
}

static int plan(const FlashArgs& a, const SeqLens* lens, int* grid, Schedule* sc) {
    SeqLens sl;
    if (a.ragged) sl = *lens;
    else sl.len[0] = a.T;
    // the schedule is planned for one workgroup per CU; the grid is then at most one per unit
    int cus = 0;
    DT_TRY(persistent_grid(0x7fffffff, &cus));
    build_schedule(a, sl, cus, true, sc, true);
    *grid = sc->n_units < cus ? sc->n_units : cus;
    return DT_OK;
}

int flash_fwd_split_items(const FlashArgs& a, const SeqLens* lens, int* n_items) {
    int grid = 0;
    Schedule sc;
    DT_TRY(plan(a, lens, &grid, &sc));
    *n_items = sc.n_slots;
    return DT_OK;
}

int launch_flash_fwd_bf16(const FlashArgs& a, const SeqLens* lens, hipStream_t stream) {
    if (a.ldk != a.ldv) return set_error(DT_ERR_UNSUPPORTED, "bf16 kernel needs equal K and V row strides");
    if ((int64_t)a.T * a.ldk * 2 >= ((int64_t)1 << 31) || (int64_t)a.T * a.ldq * 2 >= ((int64_t)1 << 31))
        return set_error(DT_ERR_UNSUPPORTED, "Q/K/V extent of one sequence exceeds 2 GiB");
    int grid = 0;
    Schedule sc;
    DT_TRY(plan(a, lens, &grid, &sc));
    if (sc.n_slots > 0 && (sc.n_slots > a.split_slots || !a.split_ws || !a.split_cnt)) {  // no room: whole items
        SeqLens sl;
        if (a.ragged) sl = *lens;
        else sl.len[0] = a.T;
        build_schedule(a, sl, grid, false, &sc, true);
        grid = sc.n_units < grid ? sc.n_units : grid;
    }
    hipLaunchKernelGGL(flash_fwd_bf16_kernel, dim3(grid), dim3(kThreads), 0, stream, a, sc);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
