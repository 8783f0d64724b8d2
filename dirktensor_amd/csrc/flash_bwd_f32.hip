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
// in both kernels. Each workgroup owns one block; the grid lists the blocks in
// decreasing causal cost, so the hardware's first-free-CU dispatch runs the
// longest blocks first. With more than one block per CU and pass the dS path
// replaces the dQ kernel: the dK/dV kernel also stores dS (fp32) and
// flash_bwd_dq_ds forms dQ = dS K from it (5 products per tile pair instead of 7).
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
// Tiles move from HBM straight into LDS with buffer_load ... lds, double-buffered
// (the next tile streams in while the current one is used; one barrier per
// tile). LDS rows are 512 bytes (128 floats), unpadded; the 16-byte chunk c of
// row r is stored at chunk position c ^ (r & 15), so the row-wise reads of the
// head-dimension products (16 rows, one chunk each) are conflict-free; the
// column reads of the other products (two rows, 8 chunks each) meet in pairs
// of banks (LDS bandwidth is far from the limit at fp32 MFMA rates). Every LDS
// operand goes through a four-deep register ring, three reads ahead of the
// MFMAs that consume it.

#include "dt_internal.h"

#include <climits>

#include <type_traits>
#include <utility>

namespace dt {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kD = 128;
constexpr int kTile = 64;
constexpr int kRowBytes = kD * 4;              // one LDS row, unpadded
constexpr int kTileBytes = kTile * kRowBytes;  // 32 KB
constexpr int kBlk = 128;
constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBufferDword3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ floatx16 mfma(float a, float b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 zero16() {
    floatx16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.0f;
    return z;
}

template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
// calls f(std::integral_constant<int, I>{}) for I = 0 .. N-1 (compile-time unrolled)
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}
// keeps each group of MFMAs with the LDS reads issued beside it: the scheduler may not move work across
#define DT_BUNDLE_END __builtin_amdgcn_sched_barrier(0)

// x as an opaque value at this point: address arithmetic derived from it is done where it is used instead
// of being hoisted out of the tile loop into long-lived registers
__device__ __forceinline__ int fresh(int x) {
    asm volatile("" : "+v"(x));
    return x;
}
// byte offset of float x of row r in a swizzled LDS tile
__device__ __forceinline__ int swz(int r) { return r & 15; }

// Buffer descriptor over [base, base + bytes): loads at or past the end return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferDword3);
}
// LDS DMA issued through inline assembly: the compiler does not track these loads, so it does not wait
// for them before reading the other LDS stage; stage_barrier() waits for them before any wave reads the
// stage they fill. M0 (an operand bound to M0) holds the wave-uniform LDS destination; lane i writes 16
// (or 4) bytes at M0 + 16*i (4*i).
// The compiler cannot insert the wait states the hardware needs before these instructions (5 after a VALU
// write of an SGPR they read, such as a v_readlane reload of the descriptor; 1 after an SALU write of M0),
// since it does not see inside the asm: s_nop 4 provides them.
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_void*)p; }
__device__ __forceinline__ void dma16(uint32_t lds, uint32_t voff, __amdgpu_buffer_rsrc_t r) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4(uint32_t lds, uint32_t voff, __amdgpu_buffer_rsrc_t r) {
    asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds) : "memory");
}
// this wave's LDS DMA and LDS accesses are complete before any wave passes it
__device__ __forceinline__ void stage_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// rows r0 .. T-1 of a [T][ld] fp32 tensor -> one LDS tile (rows past T arrive as zeros). Instruction n
// of wave w fills LDS rows 2*(4n + w) and 2*(4n + w) + 1 (1 KB, 16 bytes per lane at chunk position
// lane % 32); the lane fetches the chunk the swizzle puts there. The row offsets are formed here from
// one opaque value rather than kept in registers across the tile loop.
__device__ __forceinline__ void dma_tile(uint8_t* tile, const float* base, int r0, int T, int ld, int lane, int wave) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(base + (int64_t)r0 * ld, (uint32_t)(T - r0) * (uint32_t)ld * 4u);
    const uint32_t l0 = __builtin_amdgcn_readfirstlane(lds_addr(tile + wave * 1024));
    const int r_lane = fresh(2 * wave + (lane >> 5));  // row of instruction 0; instruction n adds 8n
    const int pos = lane & 31;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
        const int row = r_lane + 8 * n;
        dma16(l0 + 4096 * n, (uint32_t)((row * ld + 4 * (pos ^ swz(row))) * 4), r);
    }
}
// 64 floats t0 .. t0+63 of a [T] row -> LDS (one wave; entries past T arrive as zeros)
__device__ __forceinline__ void dma_stats(float* dst, const float* base, int t0, int T, int lane) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(base + t0, (uint32_t)(T - t0) * 4u);
    dma4(__builtin_amdgcn_readfirstlane(lds_addr(dst)), (uint32_t)lane * 4u, r);
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
// the LDS tile's rows as M and a register row half as the B operand. Two such products (tiles x and y,
// register halves fx and fy) run as two interleaved accumulator chains, so consecutive MFMAs never
// depend on each other; the LDS operands go through a three-deep register ring, two reads ahead of
// the MFMAs that consume them.
__device__ __forceinline__ void dot_rows2(floatx16& cx, floatx16& cy, const uint8_t* tx, const uint8_t* ty, int blk,
                                          int ln, int hh, const float (&fx)[64], const float (&fy)[64]) {
    cx = zero16();
    cy = zero16();
    // chunk 16*hh + j of row r = 32*blk + ln sits at position 16*hh + (j ^ (ln & 15))
    const int base = fresh((32 * blk + ln) * kRowBytes + 256 * hh) | ((ln & 15) << 4);
    auto rd = [&](const uint8_t* t, int j) { return *reinterpret_cast<const float4*>(t + (base ^ (j << 4))); };
    float4 x[3], y[3];
    x[0] = rd(tx, 0);
    y[0] = rd(ty, 0);
    x[1] = rd(tx, 1);
    y[1] = rd(ty, 1);
    static_for<16>([&](auto J) {
        constexpr int j = decltype(J)::value;
        if constexpr (j + 2 < 16) {
            x[(j + 2) % 3] = rd(tx, j + 2);
            y[(j + 2) % 3] = rd(ty, j + 2);
        }
        const float4 u = x[j % 3], v = y[j % 3];
        cx = mfma(u.x, fx[4 * j], cx);
        cy = mfma(v.x, fy[4 * j], cy);
        cx = mfma(u.y, fx[4 * j + 1], cx);
        cy = mfma(v.y, fy[4 * j + 1], cy);
        cx = mfma(u.z, fx[4 * j + 2], cx);
        cy = mfma(v.z, fy[4 * j + 2], cy);
        cx = mfma(u.w, fx[4 * j + 3], cx);
        cy = mfma(v.w, fy[4 * j + 3], cy);
        DT_BUNDLE_END;
    });
}
// acc[db] += sum over the 64 tile rows of tile[row][32*db + ln] * w[blk][i], row = 32*blk + 8*(i/4) + 4*hh + i%4
// (step t = 16*blk + i reads its four LDS values, one per db, three steps ahead)
__device__ __forceinline__ void acc_cols(floatx16 (&acc)[4], const uint8_t* tile, int ln, int hh, const floatx16 (&w)[2]) {
    // float 32*db + ln of row r = 32*(t/16) + 8*((t%16)/4) + 4*hh + t%4 is chunk 8*db + ln/4, at position
    // (8*db + ln/4) ^ (r & 15) = 8*(db ^ ((t/4) & 1)) + ((ln/4) ^ (4*hh + t%4))
    const int lane_part = fresh((hh * 4) * kRowBytes + 4 * (ln & 3));
    const int cx = fresh((ln >> 2) ^ (4 * hh));
    auto rd = [&](int t) {
        const int i = t & 15;
        const int r0 = 32 * (t >> 4) + 8 * (i / 4) + (i % 4);  // row without the lane half
        const int g = (t >> 2) & 1;
        const uint8_t* row = tile + r0 * kRowBytes + lane_part + ((cx ^ (t & 3)) << 4);
        return make_float4(*reinterpret_cast<const float*>(row + ((0 ^ g) << 7)),
                           *reinterpret_cast<const float*>(row + ((1 ^ g) << 7)),
                           *reinterpret_cast<const float*>(row + ((2 ^ g) << 7)),
                           *reinterpret_cast<const float*>(row + ((3 ^ g) << 7)));
    };
    float4 x[4];
    x[0] = rd(0);
    x[1] = rd(1);
    x[2] = rd(2);
    static_for<32>([&](auto Tc) {
        constexpr int t = decltype(Tc)::value;
        if constexpr (t + 3 < 32) x[(t + 3) & 3] = rd(t + 3);
        const float4 v = x[t & 3];
        const float wv = w[t >> 4][t & 15];
        acc[0] = mfma(v.x, wv, acc[0]);
        acc[1] = mfma(v.y, wv, acc[1]);
        acc[2] = mfma(v.z, wv, acc[2]);
        acc[3] = mfma(v.w, wv, acc[3]);
        DT_BUNDLE_END;
    });
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
// LDS stage: Q tile, dO tile, and the tile rows' lse2 and delta
struct DkdvStage {
    uint8_t q[kTileBytes];
    uint8_t g[kTileBytes];
    float lse2[kTile];
    float delta[kTile];
};

// dS workspace blocks (the dS path): 128 key rows of 256 bytes (the 64 queries of a query tile); 16-byte
// chunk c of a row holds queries 4c .. 4c+3 (one dK/dV lane's four consecutive accumulator rows) and sits at
// position c ^ (8 * ((row >> 2) & 1)), so the dQ pass's reads of rows r and r + 4 (its two lane halves)
// fall in different banks.
constexpr int kDsRowBytes = 256;
constexpr int kDsBlockBytes = kBlk * kDsRowBytes;  // 32 KB
constexpr int kDsHalfBytes = kTile * kDsRowBytes;  // the rows of one 64-key tile: 16 KB

// dK and dV of key block kb_own of (batch, head) bh; kEmitDs: also dS -> the dS workspace
template <bool kEmitDs>
__device__ __forceinline__ void dkdv_block(const FlashBwdArgs& a, int kb_own, int bh, DkdvStage (&stg)[2]) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 31;
    const int hh = lane >> 5;
    const int T = a.T;
    const float c = a.scale * kLog2e;

    const int b = bh / a.H, h = bh % a.H;

    const float* Qg = static_cast<const float*>(a.q) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Kg = static_cast<const float*>(a.k) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Vg = static_cast<const float*>(a.v) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Gg = static_cast<const float*>(a.d_o) + (int64_t)b * T * a.ld_o + (int64_t)h * kD;
    const float* lse2g = a.lse2 + (int64_t)bh * T;
    const float* deltag = a.delta + (int64_t)bh * T;
    float* dKg = static_cast<float*>(a.d_k) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;
    float* dVg = static_cast<float*>(a.d_v) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;

    // Q, dO, lse2 and delta rows q0 .. q0+63 -> stage s
    auto fetch = [&](DkdvStage& s, int q0) {
        dma_tile(s.q, Qg, q0, T, a.ld_qkv, lane, wave);
        dma_tile(s.g, Gg, q0, T, a.ld_o, lane, wave);
        if (wave == 0) dma_stats(s.lse2, lse2g, q0, T, lane);
        if (wave == 1) dma_stats(s.delta, deltag, q0, T, lane);
    };

    {
        const int kb = kb_own;
        const int kw = kb * kBlk + 32 * wave;
        const int key = kw + ln;

        const int q_begin = a.causal ? kb * kBlk : 0;
        const int n_steps = (T - q_begin + kTile - 1) / kTile;
        fetch(stg[0], q_begin);  // both stages are free: the previous block ended with a barrier

        // dS stores: this key block's blocks of the workspace; lane row 32*wave + ln
        uint8_t* ds_base = nullptr;
        if constexpr (kEmitDs) {
            const BwdDsLayout lay(T, a.causal);
            ds_base = static_cast<uint8_t*>(a.ds_ws) + (uint64_t)(bh * lay.per_head() + lay.block_offset(kb)) * kDsBlockBytes;
        }
        const int ds_row = (32 * wave + ln) * kDsRowBytes;
        const int ds_xs = 8 * ((ln >> 2) & 1);

        float kf[64], vf[64];
        load_half_row(kf, Kg, key, T, a.ld_qkv, hh);
        load_half_row(vf, Vg, key, T, a.ld_qkv, hh);
        floatx16 dv[4], dk[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            dv[db] = zero16();
            dk[db] = zero16();
        }
        stage_barrier();
        // kMask: the tile may hold masked elements; kSkip: the wave may have no query of the tile to take
        auto tile = [&](auto MASK, auto SKIP, int it) __attribute__((always_inline)) {
            constexpr bool kMask = decltype(MASK)::value;
            const int q0 = q_begin + it * kTile;
            const DkdvStage& s = stg[it & 1];
            if (it + 1 < n_steps) fetch(stg[(it + 1) & 1], q0 + kTile);
            if (!(decltype(SKIP)::value && a.causal && q0 + kTile - 1 < kw)) {
                // (the dQ pass never reads the dS of a skipped tile and wave: all of it is masked); with dS
                // stored, keys past T are masked too (their dS would otherwise be exp2(-lse2) (-delta))
                const bool need_mask = (a.causal && q0 < kw + 31) || (kEmitDs && kw + 31 >= T);
                // masking without branches: element i of query block qb (query q0 + 32*qb + 4*hh + off_i,
                // off_i = 8*(i/4) + i%4) is masked when dmask[qb] > off_i, i.e. when key > query (causal) or,
                // with dS stored, key >= T; INT_MIN when nothing in the tile is masked
                int dmask[2];
#pragma unroll
                for (int qb = 0; qb < 2; ++qb)
                    dmask[qb] = !need_mask              ? INT_MIN
                                : (kEmitDs && key >= T) ? INT_MAX
                                : a.causal              ? key - (q0 + 32 * qb + 4 * hh)
                                                        : INT_MIN;
                floatx16 sc[2], dp[2];
                // S = Q K^T (raw), dP = dO V^T (two query blocks; explicit calls keep every index static)
                dot_rows2(sc[0], dp[0], s.q, s.g, 0, ln, hh, kf, vf);
                dot_rows2(sc[1], dp[1], s.q, s.g, 1, ln, hh, kf, vf);
                // P and dS overwrite S and dP in place
#pragma unroll
                for (int qb = 0; qb < 2; ++qb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int qi = 32 * qb + 8 * (i / 4) + 4 * hh + (i % 4);
                        float pv = __builtin_amdgcn_exp2f(sc[qb][i] * c - s.lse2[qi]);
                        if constexpr (kMask) pv = dmask[qb] > 8 * (i / 4) + (i % 4) ? 0.0f : pv;
                        sc[qb][i] = pv;
                        dp[qb][i] = pv * (dp[qb][i] - s.delta[qi]);
                    }
                if constexpr (kEmitDs) {  // dS: chunk 8*qb + 2*g + hh of the lane's key row
                    uint8_t* blk = ds_base + (size_t)(it * kDsBlockBytes);
#pragma unroll
                    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
                        for (int g = 0; g < 4; ++g)
                            *reinterpret_cast<float4*>(blk + ds_row + (((8 * qb + 2 * g + hh) ^ ds_xs) << 4)) =
                                make_float4(dp[qb][4 * g], dp[qb][4 * g + 1], dp[qb][4 * g + 2], dp[qb][4 * g + 3]);
                }
                acc_cols(dv, s.g, ln, hh, sc);  // dV^T += dO^T P
                acc_cols(dk, s.q, ln, hh, dp);  // dK^T += Q^T dS
            }
            stage_barrier();  // stage it&1 is free for the tile after next; tile it+1 has landed
        };
        // Tiles 0 and 1 hold the diagonal (causal masks; under causality waves 2-3 have no query of tile 0);
        // from tile 2 on nothing is masked, so that loop is compiled without the selects and the skip (the
        // same values: dmask is INT_MIN there). The kernel that stores dS keeps one loop: peeled, it spilled.
        using True_ = std::true_type;
        using False_ = std::false_type;
        if constexpr (kEmitDs) {
            for (int it = 0; it < n_steps; ++it) tile(True_{}, True_{}, it);
        } else {
            tile(True_{}, True_{}, 0);
            if (n_steps > 1) tile(True_{}, False_{}, 1);
            for (int it = 2; it < n_steps; ++it) tile(False_{}, False_{}, it);
        }
        if (key < T) {
            store_rows(dKg, key, a.ld_grad, hh, dk, a.scale);  // dS carries the reference's scale (:293)
            store_rows(dVg, key, a.ld_grad, hh, dv, 1.0f);
        }
    }
}

// ------------------------------------------------------------------------------------------------ dQ
// LDS stage: K tile, V tile
struct DqStage {
    uint8_t k[kTileBytes];
    uint8_t v[kTileBytes];
};

// dQ of query block qb_own of (batch, head) bh
__device__ __forceinline__ void dq_block(const FlashBwdArgs& a, int qb_own, int bh, DqStage (&stg)[2]) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 31;
    const int hh = lane >> 5;
    const int T = a.T;
    const float c = a.scale * kLog2e;

    const int b = bh / a.H, h = bh % a.H;

    const float* Qg = static_cast<const float*>(a.q) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Kg = static_cast<const float*>(a.k) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Vg = static_cast<const float*>(a.v) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const float* Gg = static_cast<const float*>(a.d_o) + (int64_t)b * T * a.ld_o + (int64_t)h * kD;
    float* dQg = static_cast<float*>(a.d_q) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;

    // K and V rows k0 .. k0+63 -> stage s
    auto fetch = [&](DqStage& s, int k0) {
        dma_tile(s.k, Kg, k0, T, a.ld_qkv, lane, wave);
        dma_tile(s.v, Vg, k0, T, a.ld_qkv, lane, wave);
    };

    {
        const int qb = qb_own;
        const int qw = qb * kBlk + 32 * wave;
        const int q = qw + ln;

        const int k_end = a.causal ? min(qb * kBlk + kBlk, T) : T;
        const int n_steps = (k_end + kTile - 1) / kTile;
        fetch(stg[0], 0);  // both stages are free: the previous block ended with a barrier

        float qf[64], gf[64];
        load_half_row(qf, Qg, q, T, a.ld_qkv, hh);
        load_half_row(gf, Gg, q, T, a.ld_o, hh);
        const float lse2 = q < T ? a.lse2[(int64_t)bh * T + q] : 0.0f;
        const float delta = q < T ? a.delta[(int64_t)bh * T + q] : 0.0f;
        const int lim = a.causal ? min(q, T - 1) : T - 1;
        floatx16 dq[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) dq[db] = zero16();

        stage_barrier();
        // kGen: the tile may hold masked keys, or none the wave's queries see
        auto tile = [&](auto GEN, int it) __attribute__((always_inline)) {
            constexpr bool kGen = decltype(GEN)::value;
            const int k0 = it * kTile;
            const DqStage& s = stg[it & 1];
            if (it + 1 < n_steps) fetch(stg[(it + 1) & 1], k0 + kTile);
            if (!(kGen && a.causal && k0 > qw + 31)) {
                const bool need_mask = (a.causal && k0 + kTile - 1 > qw) || k0 + kTile > T;
                // masking without branches: element i of key block kb (key k0 + 32*kb + 4*hh + off_i, off_i =
                // 8*(i/4) + i%4) is masked when off_i > emask[kb], i.e. when key > lim
                int emask[2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) emask[kb] = need_mask ? lim - (k0 + 32 * kb + 4 * hh) : INT_MAX;
                floatx16 sc[2], dp[2];
                // S^T = K Q^T (raw), dP^T = V dO^T (two key blocks; explicit calls keep every index static)
                dot_rows2(sc[0], dp[0], s.k, s.v, 0, ln, hh, qf, gf);
                dot_rows2(sc[1], dp[1], s.k, s.v, 1, ln, hh, qf, gf);
                floatx16 ds[2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        float pv = __builtin_amdgcn_exp2f(sc[kb][i] * c - lse2);
                        if constexpr (kGen) pv = 8 * (i / 4) + (i % 4) > emask[kb] ? 0.0f : pv;
                        ds[kb][i] = pv * (dp[kb][i] - delta);
                    }
                acc_cols(dq, s.k, ln, hh, ds);  // dQ^T += K^T dS^T
            }
            stage_barrier();  // stage it&1 is free for the tile after next; tile it+1 has landed
        };
        // Tiles 0 .. n_plain-1 need no mask (every key at or before the wave's first query and before T); the
        // rest (the diagonal under causality, the tile past T) take the selects and, past the wave's queries,
        // nothing. Two loops, so the first is compiled without them (the same values: emask is INT_MAX).
        const int k_plain = a.causal ? min(qw + 1, T) : T;
        const int n_plain = min(max(k_plain, 0) / kTile, n_steps);
        int it = 0;
        for (; it < n_plain; ++it) tile(std::false_type{}, it);
        for (; it < n_steps; ++it) tile(std::true_type{}, it);
        if (q < T) store_rows(dQg, q, a.ld_grad, hh, dq, a.scale);
    }
}

// ------------------------------------------------------------------------------------------------ dQ from dS
// LDS stage: a 64-key tile of K and the dS rows of those keys for the block's two 64-query tiles
struct DsqStage {
    uint8_t k[kTileBytes];
    uint8_t ds[2][kDsHalfBytes];
};

// dQ of query block qb_own of (batch, head) bh from the dS the dK/dV pass stored: per 64-key tile
// dQ^T += K^T dS^T, the A operand from the K tile as in acc_cols and the B operand (one key and query per
// lane and step) read from the dS tile.
__device__ __forceinline__ void dq_ds_block(const FlashBwdArgs& a, int qb_own, int bh, DsqStage (&stg)[2]) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 31;
    const int hh = lane >> 5;
    const int T = a.T;
    const int b = bh / a.H, h = bh % a.H;
    const float* Kg = static_cast<const float*>(a.k) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    float* dQg = static_cast<float*>(a.d_q) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;
    const BwdDsLayout lay(T, a.causal);
    const uint8_t* ds_head = static_cast<const uint8_t*>(a.ds_ws) + (uint64_t)(bh * lay.per_head()) * kDsBlockBytes;

    const int qw = qb_own * kBlk + 32 * wave;  // the wave's first query
    const int q = qw + ln;
    const int qt0 = 2 * qb_own;                // the block's first 64-query tile
    const int n_qt = min(2, lay.nqt - qt0);
    const int k_end = a.causal ? min(qb_own * kBlk + kBlk, T) : T;
    const int n_steps = (k_end + kTile - 1) / kTile;

    // K rows k0 .. k0+63 and their dS rows of the block's query tiles -> stage s (the dS rows as stored:
    // instruction n of wave w moves 1 KB of each 16 KB half)
    auto fetch = [&](DsqStage& s, int k0) {
        dma_tile(s.k, Kg, k0, T, a.ld_qkv, lane, wave);
        const int kb = k0 / kBlk;
        const uint8_t* blk = ds_head + (uint64_t)(lay.block_offset(kb) + (qt0 - lay.first_tile(kb))) * kDsBlockBytes;
        const __amdgpu_buffer_rsrc_t r = make_rsrc(blk, (uint32_t)n_qt * kDsBlockBytes);
        const uint32_t rows = (uint32_t)((k0 / kTile) & 1) * kDsHalfBytes;  // this tile's rows of the key block
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                const uint32_t chunk = (uint32_t)((n * 4 + wave) * 64);  // 16-byte chunks of a 16 KB half
                dma16(__builtin_amdgcn_readfirstlane(lds_addr(s.ds[t] + chunk * 16)),
                      (uint32_t)t * kDsBlockBytes + rows + (chunk + (uint32_t)lane) * 16u, r);
            }
    };

    // the B operand of step t (t = 16*blk + i): dS of key row 32*blk + 8*(i/4) + 4*hh + i%4 and this lane's
    // query (column 32*(wave & 1) + ln of query tile wave / 2); that row's (row >> 2) & 1 is hh, so the
    // chunk's position is a constant of the lane
    const int qcol = 32 * (wave & 1) + ln;
    const int ds_lane = (wave >> 1) * kDsHalfBytes + 4 * hh * kDsRowBytes + (((qcol >> 2) ^ (8 * hh)) << 4) + 4 * (qcol & 3);
    floatx16 dq[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) dq[db] = zero16();

    // the tiles this wave multiplies: 0 .. n_use-1 (no query of the wave, or every key of a later tile
    // after its queries under causality, leaves the rest to the other waves); the rest only fetch and wait,
    // in a loop of their own (a product skipped inside the loop made the compiler copy the accumulators)
    const int n_use = q - ln >= T ? 0 : (a.causal ? min(n_steps, (qw + 31) / kTile + 1) : n_steps);
    fetch(stg[0], 0);
    stage_barrier();
    int it = 0;
    for (; it < n_use; ++it) {
        const int k0 = it * kTile;
        const DsqStage& s = stg[it & 1];
        if (it + 1 < n_steps) fetch(stg[(it + 1) & 1], k0 + kTile);
        {
            // the second 32 keys are all after the wave's queries under causality: their dS was not stored
            const bool second = !a.causal || k0 + 32 <= qw + 31;
            floatx16 w[2];
#pragma unroll
            for (int blk = 0; blk < 2; ++blk)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int r = 32 * blk + 8 * (i / 4) + (i % 4);  // the key row without the lane half
                    const float x = *reinterpret_cast<const float*>(s.ds[0] + ds_lane + r * kDsRowBytes);
                    w[blk][i] = (blk == 0 || second) ? x : 0.0f;
                }
            acc_cols(dq, s.k, ln, hh, w);  // dQ^T += K^T dS^T
        }
        stage_barrier();  // stage it&1 is free for the tile after next; tile it+1 has landed
    }
    for (; it < n_steps; ++it) {
        if (it + 1 < n_steps) fetch(stg[(it + 1) & 1], (it + 1) * kTile);
        stage_barrier();
    }
    if (q < T) store_rows(dQg, q, a.ld_grad, hh, dq, a.scale);
}

// One 128-row block per workgroup, listed in decreasing causal cost, so that the hardware, which hands
// the next workgroup to the first CU that frees up, runs a longest-first schedule.
// pass = 0 (dK/dV) or 1 (dQ): one pass per launch; workgroup BH*j + bh takes, for (batch, head) bh,
//   key block j (dK/dV; key block 0 sees every query tile) or query block n-1-j (dQ).
// pass = 2: both passes in one launch; workgroup 2*BH*j + BH*kind + bh takes the dK/dV of key block j
//   (kind 0) or the dQ of query block n-1-j (kind 1), which see the same number of tiles under
//   causality, so the list stays in decreasing cost and the two passes share the CUs.
union BwdLds {
    DkdvStage kv[2];
    DqStage q[2];
};

__global__ __launch_bounds__(kThreads, 1) void flash_bwd_f32_kernel(FlashBwdArgs a, int pass) {
    __shared__ __attribute__((aligned(1024))) BwdLds lds;
    const int BH = a.B * a.H;
    const int n = (a.T + kBlk - 1) / kBlk;
    const int j = (int)blockIdx.x / (pass == 2 ? 2 * BH : BH);
    const int kind = pass == 2 ? ((int)blockIdx.x / BH) & 1 : pass;
    const int bh = (int)blockIdx.x % BH;
    if (kind == 0) dkdv_block<false>(a, j, bh, lds.kv);
    else dq_block(a, n - 1 - j, bh, lds.q);
}

// The dS path: the dK/dV pass (workgroup BH*j + bh: key block j) storing dS, then dQ = dS K (workgroup
// BH*j + bh: query block n-1-j), both in decreasing causal cost.
__global__ __launch_bounds__(kThreads, 1) void flash_bwd_dkdv_ds_f32_kernel(FlashBwdArgs a) {
    __shared__ __attribute__((aligned(1024))) DkdvStage st[2];
    const int BH = a.B * a.H;
    dkdv_block<true>(a, (int)blockIdx.x / BH, (int)blockIdx.x % BH, st);
}
__global__ __launch_bounds__(kThreads, 1) void flash_bwd_dq_ds_f32_kernel(FlashBwdArgs a) {
    __shared__ __attribute__((aligned(1024))) DsqStage st[2];
    const int BH = a.B * a.H;
    const int n = (a.T + kBlk - 1) / kBlk;
    dq_ds_block(a, n - 1 - (int)blockIdx.x / BH, (int)blockIdx.x % BH, st);
}

}  // namespace

int launch_flash_bwd_f32(const FlashBwdArgs& a, hipStream_t stream) {
    const int64_t ld = a.ld_qkv > a.ld_o ? a.ld_qkv : a.ld_o;
    if ((int64_t)a.T * ld * 4 >= ((int64_t)1 << 31))
        return set_error(DT_ERR_UNSUPPORTED, "Q/K/V/dO extent of one sequence exceeds 2 GiB");
    DT_TRY(launch_flash_bwd_prep(a, 0, stream));
    const int64_t blocks = (int64_t)((a.T + kBlk - 1) / kBlk) * a.B * a.H;  // per pass, one per workgroup
    if (2 * blocks > 0x7fffffff) return set_error(DT_ERR_UNSUPPORTED, "too many workgroups");
    if (a.ds_ws) {  // dS stored by the dK/dV pass, dQ = dS K
        hipLaunchKernelGGL(flash_bwd_dkdv_ds_f32_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
        DT_HIP_TRY(hipGetLastError());
        hipLaunchKernelGGL(flash_bwd_dq_ds_f32_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
        DT_HIP_TRY(hipGetLastError());
        return DT_OK;
    }
    int cus = 0;
    DT_TRY(persistent_grid(0x7fffffff, &cus));
    if (blocks <= cus) {  // the passes share one launch (at most one block per CU and pass)
        hipLaunchKernelGGL(flash_bwd_f32_kernel, dim3((unsigned)(2 * blocks)), dim3(kThreads), 0, stream, a, 2);
        DT_HIP_TRY(hipGetLastError());
    } else {
        for (int pass = 0; pass < 2; ++pass) {
            hipLaunchKernelGGL(flash_bwd_f32_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a, pass);
            DT_HIP_TRY(hipGetLastError());
        }
    }
    return DT_OK;
}

}  // namespace dt
