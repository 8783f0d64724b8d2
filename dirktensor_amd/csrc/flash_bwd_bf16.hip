// Causal flash attention backward, bf16 MFMA mode, for gfx950 (CDNA4).
//
// Replaces flash_attention_backward (FlashAttention.cpp:185-359) with bf16
// Q/K/V/O/dO/dQ/dK/dV, fp32 accumulation and fp32 P / dS arithmetic.
//
// The reference walks (query block, key block) pairs and accumulates all three
// gradients from each pair; dK and dV rows receive contributions from many
// query blocks and dQ rows from many key blocks. Here each gradient has one
// owner, so nothing is accumulated through memory and the result does not
// depend on scheduling:
//   * flash_bwd_dkdv: a workgroup owns 128 keys of one (batch, head), 32 per
//     wave, holds their K and V fragments in registers and streams 64-query
//     tiles of Q and dO (plus the rows' lse2 and delta) through LDS. Per tile
//     a wave forms S = Q K^T and dP = dO V^T for its keys, then
//     P = exp2(S c - lse2) and dS = P (dP - delta), and accumulates
//     dV^T += dO^T P and dK^T += Q^T dS.
//   * flash_bwd_dq: a workgroup owns 128 queries, 32 per wave, holds their Q
//     and dO fragments in registers and streams 64-key tiles of K and V.
//     Per tile a wave forms S^T = K Q^T and dP^T = V dO^T, the same P and dS,
//     and accumulates dQ^T += K^T dS^T.
//   On this recompute path S and dP are formed in both kernels (7 MFMA
//   products per tile pair instead of the reference's 5) in exchange for no
//   atomics.
//   * The dS path (flash_bwd_dkdv_ds + flash_bwd_dq_ds, the default where each
//     pass has more than one block per CU, e.g. B*H = 16 at T = 4096): the
//     dK/dV kernel also stores the bf16 dS it forms for its dK product to a
//     workspace, and the dQ kernel computes dQ = dS K from it, so a tile pair
//     takes 5 products, still with one owner per gradient row and no atomics.
// Causality (FlashAttention.cpp:247, 265-268) limits the dK/dV kernel to query
// tiles at or after its keys and the dQ kernel to key tiles at or before its
// queries. Each workgroup owns one 128-row block; the grid lists the blocks in
// decreasing causal cost, and the hardware gives the next workgroup to the first
// CU that frees up, which schedules the longest blocks first and fills the tail
// with the short ones (at T = 6144 the longest CU then carries 81 tile steps
// for an average of 73.5, where fixed pairs of blocks j and n-1-j carried 98).
//
// MFMA operand layouts (v_mfma_f32_32x32x16_bf16): the A operand is a 32-row
// fragment, lane l holding row l%32 and k elements 8*(l/32) .. +8; the B
// operand is a 32-column fragment, lane l holding column l%32 and the same k
// elements; accumulator element i of lane l is row 8*(i/4) + 4*(l/32) + i%4,
// column l%32. An accumulator can therefore feed the next product directly as
// its B operand (its rows become the k index, in that permuted order), with the
// A operand read from LDS by the gfx950 transposing read ds_read_b64_tr_b16 in
// the same permuted order; this is how P, dS (dK/dV kernel) and dS^T (dQ
// kernel) enter the second products without leaving registers.
//
// LDS tiles are 64 rows of 256 bytes, unpadded, with 16-byte chunk c of row r
// stored at c ^ swz(r), swz(r) = 4*(r & 3) + ((r >> 2) & 3): row-wise fragment
// reads and transposing reads are both free of bank conflicts. Tiles arrive
// by LDS DMA (buffer_load ... lds), double-buffered, one barrier per tile;
// buffer descriptors end at row T - 1 so rows past the sequence arrive as zeros.
// Every product reads its LDS fragments through a four-deep register ring,
// three reads ahead of the MFMA that consumes them: with one wave per SIMD
// nothing else hides an LDS round trip.

#include "dt_internal.h"

#include <climits>
#include <type_traits>
#include <utility>

namespace dt {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef short shortx8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;

constexpr int kD = 128;
constexpr int kTile = 64;                      // rows per streamed tile
constexpr int kRowBytes = 256;                 // one row of 128 bf16
constexpr int kTileBytes = kTile * kRowBytes;  // 16 KB
constexpr int kBlk = 128;                      // rows owned by a workgroup: 4 waves x 32
constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBufferDword3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

// dS workspace (the path that stores dS in the dK/dV pass and computes dQ = dS K from it). Per (batch, head)
// and 128-key block kb, one 16 KB block per 64-query tile the keys can see (tiles 2*kb .. under causality,
// all otherwise), tiles of one key block consecutive. A block holds 128 key rows of 128 bytes; a row holds
// the tile's 64 queries as 16-byte chunks, chunk c = 4*qb + 2*u + hh holding queries 32*qb + 16*u + 4*hh
// + {0..3} and then + 8 + {0..3} (one dK/dV lane's bf16 B operand of dS, stored whole), at chunk position
// c ^ (2 * (row & 3)) so that the dQ pass's transposing reads of four consecutive rows hit distinct banks.
constexpr int kDsRowBytes = 128;
constexpr int kDsBlockBytes = kBlk * kDsRowBytes;  // 16 KB
constexpr int kDsHalfBytes = kTile * kDsRowBytes;  // the rows of one 64-key tile: 8 KB


__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 r = __builtin_convertvector((floatx2){lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferDword3);
}
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ floatx16 mfma(bf16x8 a, bf16x8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
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
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// keeps each MFMA with the LDS read issued beside it: the scheduler may not move work across
#define DT_BUNDLE_END __builtin_amdgcn_sched_barrier(0)

// Row fragment r = 2*cc + blk of a tile: rows 32*blk + ln, dims 16*cc + 8*hh .. +8 (the A operand
// with the tile's rows as M). raddr[cc] is this lane's address of chunk 2*cc + hh in block 0.
__device__ __forceinline__ bf16x8 read_row(const uint8_t* tile, const uint32_t (&raddr)[8], int cc, int blk) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(tile + raddr[cc] + blk * 8192));
}
// Transposed fragment c = 8*blk + 4*u + db of a tile: rows 32*blk + 16*u + {4*hh .. +4, 8 + 4*hh .. +4}
// (the accumulator's row order) as k, dims 32*db + ln as M (two transposing reads).
__device__ __forceinline__ bf16x8 read_tr(const uint8_t* tile, const uint32_t (&taddr)[2][4], int c) {
    const int rows = (c >> 3) * 8192 + ((c >> 2) & 1) * 4096;
    const int db = c & 3;
    const shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(tile + taddr[0][db] + rows));
    const shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(tile + taddr[1][db] + rows + 2048));
    return __builtin_bit_cast(bf16x8, (shortx8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
}

// Lane addresses shared by both kernels.
struct LaneAddr {
    uint32_t raddr[8];
    uint32_t taddr[2][4];
};
__device__ __forceinline__ LaneAddr lane_addr(int lane) {
    LaneAddr A;
    const int ln = lane & 31, hh = lane >> 5;
    const int g = hh ^ swz(ln);
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) A.raddr[cc] = (uint32_t)(ln * kRowBytes + (((2 * cc) ^ g) << 4));
    // transposing reads: lane i of 16-lane group G reads row 4*hh + i/4 (+8 for the second read) of a
    // 16-row chunk, dims 32*db + 16*(G & 1) + 4*(i & 3) .. +3
    const int i16 = lane & 15;
    const int g2 = (lane >> 4) & 1;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int r = 4 * hh + (i16 >> 2) + 8 * s;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int chunk = 4 * db + 2 * g2 + ((i16 & 3) >> 1);
            A.taddr[s][db] = (uint32_t)((r - 8 * s) * kRowBytes + ((chunk ^ swz(r)) << 4) + 8 * (i16 & 1));
        }
    }
    return A;
}

// DMA offsets of a 64-row tile with row stride ld (elements): instruction i of wave w fills rows
// 16*i + 4*w + lane/16, 16 bytes per lane at chunk position lane%16, fetching the global chunk the
// swizzle puts there.
__device__ __forceinline__ void dma_offsets(uint32_t (&voff)[4], int lane, int wave, int ld) {
    const int rlo = lane >> 4;
    const int chunk = (lane & 15) ^ (4 * rlo + wave);
#pragma unroll
    for (int i = 0; i < 4; ++i) voff[i] = (uint32_t)(((16 * i + 4 * wave + rlo) * ld + 8 * chunk) * 2);
}
// LDS DMA issued through inline assembly: the compiler does not track these loads, so it does not wait
// for them before reading the other LDS stage (it cannot prove the two stages apart and otherwise
// stalls every other step on the DMA just issued). stage_barrier() waits for them explicitly before any
// wave reads the stage they fill. M0 holds the wave-uniform LDS destination (an operand bound to M0, so
// the compiler sets it and knows it changed); lane i writes 16 (or 4) bytes at M0 + 16*i (4*i).
// The compiler cannot insert the wait states the hardware needs before these instructions (5 after a VALU
// write of an SGPR they read, such as a v_readlane reload of the descriptor; 1 after an SALU write of
// M0), since it does not see inside the asm: s_nop 4 provides them.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void dma16(uint32_t lds, uint32_t voff, __amdgpu_buffer_rsrc_t r) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4(uint32_t lds, uint32_t voff, __amdgpu_buffer_rsrc_t r) {
    asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds) : "memory");
}
// rows r0 .. T-1 of a [T][ld] bf16 tensor -> one LDS tile (rows past T arrive as zeros)
__device__ __forceinline__ void dma_tile(uint8_t* tile, const uint16_t* base, int r0, int T, int ld,
                                         const uint32_t (&voff)[4], int wave) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(base + (int64_t)r0 * ld, (uint32_t)(T - r0) * (uint32_t)ld * 2u);
    const uint32_t l0 = __builtin_amdgcn_readfirstlane(lds_addr(tile + wave * 1024));
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(l0 + 4096 * i, voff[i], r);
}
// 64 floats t0 .. t0+63 of a [T] row -> LDS (one wave; entries past T arrive as zeros)
__device__ __forceinline__ void dma_stats(float* dst, const float* base, int t0, int T, int lane) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(base + t0, (uint32_t)(T - t0) * 4u);
    dma4(__builtin_amdgcn_readfirstlane(lds_addr(dst)), (uint32_t)lane * 4u, r);
}

// this wave's LDS DMA and LDS accesses are complete before any wave passes it
__device__ __forceinline__ void stage_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// one 32-row x 128 fragment set from global memory: f[cc] = X[row][16*cc + 8*hh .. +8], zeros when row >= T
__device__ __forceinline__ void load_frags(bf16x8 (&f)[8], const uint16_t* base, int row, int T, int ld, int hh) {
    if (row < T) {
        const uint16_t* p = base + (int64_t)row * ld + 8 * hh;
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) f[cc] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p + 16 * cc));
    } else {
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) f[cc] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
    }
}

// accumulator X^T (4 blocks of 32 dims x 32 rows, lane = row) * mul -> bf16 row `row` of [T][ld] at base
__device__ __forceinline__ void store_rows(uint16_t* base, int row, int ld, int hh, const floatx16 (&x)[4], float mul) {
    uint16_t* p = base + (int64_t)row * ld;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint2 w;
            w.x = pack_bf16x2(x[db][4 * g] * mul, x[db][4 * g + 1] * mul);
            w.y = pack_bf16x2(x[db][4 * g + 2] * mul, x[db][4 * g + 3] * mul);
            *reinterpret_cast<uint2*>(p + 32 * db + 8 * g + 4 * hh) = w;
        }
}

// ------------------------------------------------------------------------------------------------ dK, dV
// LDS stage: Q tile, dO tile, and the tile rows' lse2 and delta
struct DkdvStage {
    uint8_t q[kTileBytes];
    uint8_t g[kTileBytes];
    float lse2[kTile];
    float delta[kTile];
};

// dK and dV of key block kb_own of (batch, head) bh; kEmitDs: also dS -> the dS workspace
template <bool kEmitDs>
__device__ __forceinline__ void dkdv_block(const FlashBwdArgs& a, int kb_own, int bh, DkdvStage& st0, DkdvStage& st1) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 31;
    const int hh = lane >> 5;
    const int T = a.T;
    const float c = a.scale * kLog2e;

    const int b = bh / a.H, h = bh % a.H;

    const LaneAddr LA = lane_addr(lane);
    uint32_t voff_q[4], voff_g[4];
    dma_offsets(voff_q, lane, wave, a.ld_qkv);
    dma_offsets(voff_g, lane, wave, a.ld_o);

    const uint16_t* Qg = static_cast<const uint16_t*>(a.q) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const uint16_t* Kg = static_cast<const uint16_t*>(a.k) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const uint16_t* Vg = static_cast<const uint16_t*>(a.v) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const uint16_t* Gg = static_cast<const uint16_t*>(a.d_o) + (int64_t)b * T * a.ld_o + (int64_t)h * kD;
    const float* lse2g = a.lse2 + (int64_t)bh * T;
    const float* deltag = a.delta + (int64_t)bh * T;
    uint16_t* dKg = static_cast<uint16_t*>(a.d_k) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;
    uint16_t* dVg = static_cast<uint16_t*>(a.d_v) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;

    {
        const int kb = kb_own;
        const int kw = kb * kBlk + 32 * wave;  // the wave's first key
        const int key = kw + ln;               // this lane's key (the products' N index)

        bf16x8 kf[8], vf[8];
        load_frags(kf, Kg, key, T, a.ld_qkv, hh);
        load_frags(vf, Vg, key, T, a.ld_qkv, hh);
        floatx16 dv[4], dk[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            dv[db] = zero16();
            dk[db] = zero16();
        }

        const int q_begin = a.causal ? kb * kBlk : 0;
        const int n_steps = (T - q_begin + kTile - 1) / kTile;

        // dS stores: this key block's blocks of the workspace; lane row 32*wave + ln, chunk (4*qb + 2*u + hh) ^ xs
        const __amdgpu_buffer_rsrc_t ds_rsrc = [&] {
            if constexpr (kEmitDs) {
                const BwdDsLayout lay(T, a.causal);
                const uint8_t* base = static_cast<const uint8_t*>(a.ds_ws) +
                                      (uint64_t)(bh * lay.per_head() + lay.block_offset(kb)) * kDsBlockBytes;
                return make_rsrc(base, (uint32_t)n_steps * kDsBlockBytes);
            } else {
                return make_rsrc(a.ds_ws, 0u);
            }
        }();
        // unit (key row r = 32*wave + ln, store k = 2*qb + u, half hh) of a block at
        // ((((r/32)*8 + (r%32)/4)*4 + k)*4 + r%4)*2 + hh, times 16 bytes: every store instruction writes
        // eight whole 128-byte runs (four keys' two halves), and so does every read of the dQ pass's DMA
        const uint32_t ds_lane = (uint32_t)(((wave * 8 + (ln >> 2)) * 32 + (ln & 3) * 2 + hh) * 16);

        auto dma = [&](DkdvStage& s, int q0) {
            dma_tile(s.q, Qg, q0, T, a.ld_qkv, voff_q, wave);
            dma_tile(s.g, Gg, q0, T, a.ld_o, voff_g, wave);
            if (wave == 0) dma_stats(s.lse2, lse2g, q0, T, lane);
            if (wave == 1) dma_stats(s.delta, deltag, q0, T, lane);
        };
        // kMask: the tile may hold masked elements; kSkip: the wave may have no query of the tile to take
        auto step = [&](auto MASK, auto SKIP, const DkdvStage& s, DkdvStage& nxt, int q0, bool has_next)
                        __attribute__((always_inline)) {
            constexpr bool kMask = decltype(MASK)::value;
            if (has_next) dma(nxt, q0 + kTile);
            if constexpr (decltype(SKIP)::value)
                if (a.causal && q0 + kTile - 1 < kw) return;  // every query of the tile precedes the wave's keys
            // (the dQ pass never reads the dS of such a tile and wave: all of it is masked)
            // with dS stored, keys past T are masked too (their dS would otherwise be exp2(-lse2) (-delta))
            const bool need_mask = (a.causal && q0 < kw + 31) || (kEmitDs && kw + 31 >= T);
            // masking without branches: element i of query block qb (query q0 + 32*qb + 4*hh + off_i, off_i =
            // 8*(i/4) + i%4 a constant) is masked when dmask[qb] > off_i, i.e. when key > query (causal) or,
            // with dS stored, key >= T; dmask is INT_MIN when nothing in the tile is masked
            int dmask[2];
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
                dmask[qb] = !need_mask                  ? INT_MIN
                            : (kEmitDs && key >= T)     ? INT_MAX
                            : a.causal                  ? key - (q0 + 32 * qb + 4 * hh)
                                                        : INT_MIN;
            // One software-pipelined sequence of 64 bundles (one LDS fragment read three ahead + one MFMA
            // each), the P / dS arithmetic of one 32-query block riding on the MFMAs of the next phase so
            // that it issues while the matrix pipe works:
            //   bundles  0..15  S and dP of queries 0..31   (fragment f = b: Q / dO rows)
            //   bundles 16..31  S and dP of queries 32..63; P, dS of queries 0..31, one element per bundle
            //   bundles 32..63  dV^T += dO^T P, dK^T += Q^T dS (fragment f = b: dO^T / Q^T); P, dS of
            //                   queries 32..63 in bundles 32..47
            // Row fragment f < 32: 16*qb + 2*cc + w (w = 0: Q for S, 1: dO for dP); transposed fragment
            // f >= 32: 2*ci + w with ci = 8*qb + 4*u + db (w = 0: dO^T for dV, 1: Q^T for dK).
            // Element i of block qb is query q0 + 32*qb + 8*(i/4) + 4*hh + i%4.
            // the rows' lse2 and delta of query block qb, read from LDS a few bundles before block qb's P and dS
            float Lr[2][16], Dr[2][16];
            auto load_stats = [&](int qb) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int qi = 32 * qb + 8 * g + 4 * hh;
                    const float4 L4 = *reinterpret_cast<const float4*>(&s.lse2[qi]);
                    const float4 D4 = *reinterpret_cast<const float4*>(&s.delta[qi]);
                    Lr[qb][4 * g] = L4.x, Lr[qb][4 * g + 1] = L4.y, Lr[qb][4 * g + 2] = L4.z, Lr[qb][4 * g + 3] = L4.w;
                    Dr[qb][4 * g] = D4.x, Dr[qb][4 * g + 1] = D4.y, Dr[qb][4 * g + 2] = D4.z, Dr[qb][4 * g + 3] = D4.w;
                }
            };
            floatx16 sc[2], dp[2];
            float p[2][16], ds[2][16];
            bf16x8 pb[2][2], dsb[2][2];
            auto rd = [&](int f) {
                if (f < 32) return read_row((f & 1) ? s.g : s.q, LA.raddr, (f >> 1) & 7, f >> 4);
                return read_tr((f & 1) ? s.q : s.g, LA.taddr, (f - 32) >> 1);
            };
            auto elem = [&](int qb, int i) {  // P = exp2(S c - lse2), dS = P (dP - delta)
                float pv = __builtin_amdgcn_exp2f(sc[qb][i] * c - Lr[qb][i]);
                if constexpr (kMask) pv = dmask[qb] > 8 * (i >> 2) + (i & 3) ? 0.0f : pv;
                p[qb][i] = pv;
                ds[qb][i] = pv * (dp[qb][i] - Dr[qb][i]);
            };
            auto pack = [&](int qb, int u) {  // bf16 B operands: elements 8u .. 8u+7
                uint32_t wp[4], wd[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    wp[e] = pack_bf16x2(p[qb][8 * u + 2 * e], p[qb][8 * u + 2 * e + 1]);
                    wd[e] = pack_bf16x2(ds[qb][8 * u + 2 * e], ds[qb][8 * u + 2 * e + 1]);
                }
                pb[qb][u] = __builtin_bit_cast(bf16x8, make_uint4(wp[0], wp[1], wp[2], wp[3]));
                dsb[qb][u] = __builtin_bit_cast(bf16x8, make_uint4(wd[0], wd[1], wd[2], wd[3]));
            };
            bf16x8 ring[4];
            ring[0] = rd(0);
            ring[1] = rd(1);
            ring[2] = rd(2);
            static_for<64>([&](auto B) {
                constexpr int b = decltype(B)::value;
                if constexpr (b == 12 || b == 28) load_stats(b >= 16);  // (all at the start: 1-2 % slower)
                if constexpr (b + 3 < 64) ring[(b + 3) & 3] = rd(b + 3);
                if constexpr (b < 32) {
                    constexpr int qb = b >> 4, cc = (b >> 1) & 7;
                    if constexpr (b & 1) dp[qb] = mfma(ring[b & 3], vf[cc], cc == 0 ? zero16() : dp[qb]);
                    else sc[qb] = mfma(ring[b & 3], kf[cc], cc == 0 ? zero16() : sc[qb]);
                } else {
                    constexpr int ci = (b - 32) >> 1;
                    if constexpr (b & 1) dk[ci & 3] = mfma(ring[b & 3], dsb[ci >> 3][(ci >> 2) & 1], dk[ci & 3]);
                    else dv[ci & 3] = mfma(ring[b & 3], pb[ci >> 3][(ci >> 2) & 1], dv[ci & 3]);
                }
                if constexpr (b >= 16 && b < 32) elem(0, b - 16);
                if constexpr (b >= 32 && b < 48) elem(1, b - 32);
                if constexpr (b == 23 || b == 31) pack(0, b == 31);
                if constexpr (b == 39 || b == 47) pack(1, b == 47);
                if constexpr (kEmitDs && (b == 24 || b == 32 || b == 40 || b == 48)) {
                    constexpr int qb = (b - 24) >> 4, u = ((b - 24) >> 3) & 1;
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dsb[qb][u]), ds_rsrc,
                                                          ds_lane + (uint32_t)((2 * qb + u) * 128),
                                                          (int)((q0 - q_begin) / kTile) * kDsBlockBytes, 0);
                }
                DT_BUNDLE_END;
            });
        };

        using True_ = std::true_type;
        using False_ = std::false_type;
        dma(st0, q_begin);
        stage_barrier();
        // Tiles 0 and 1 hold the diagonal (causal masks; under causality waves 2-3 have no query of tile 0).
        // From tile 2 on nothing is masked but, with dS stored, the keys past T, a condition fixed per wave:
        // the loop is compiled without the selects when it is false (the same values: dmask is INT_MIN).
        step(True_{}, True_{}, st0, st1, q_begin, 1 < n_steps);
        stage_barrier();
        if (n_steps > 1) {
            step(True_{}, False_{}, st1, st0, q_begin + kTile, 2 < n_steps);
            stage_barrier();
        }
        auto rest = [&](auto MASK) __attribute__((always_inline)) {
            for (int it = 2; it < n_steps; it += 2) {
                const int q0 = q_begin + it * kTile;
                step(MASK, False_{}, st0, st1, q0, it + 1 < n_steps);
                stage_barrier();
                if (it + 1 >= n_steps) break;
                step(MASK, False_{}, st1, st0, q0 + kTile, it + 2 < n_steps);
                stage_barrier();
            }
        };
        if (kEmitDs && kw + 31 >= T) rest(True_{});
        else rest(False_{});
        if (key < T) {
            store_rows(dKg, key, a.ld_grad, hh, dk, a.scale);  // dS carries the reference's scale (:293)
            store_rows(dVg, key, a.ld_grad, hh, dv, 1.0f);
        }
    }
}

// ------------------------------------------------------------------------------------------------ dQ
struct DqStage {
    uint8_t k[kTileBytes];
    uint8_t v[kTileBytes];
};

// dQ of query block qb_own of (batch, head) bh
__device__ __forceinline__ void dq_block(const FlashBwdArgs& a, int qb_own, int bh, DqStage& st0, DqStage& st1) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 31;
    const int hh = lane >> 5;
    const int T = a.T;
    const float c = a.scale * kLog2e;

    const int b = bh / a.H, h = bh % a.H;

    const LaneAddr LA = lane_addr(lane);
    uint32_t voff[4];
    dma_offsets(voff, lane, wave, a.ld_qkv);

    const uint16_t* Qg = static_cast<const uint16_t*>(a.q) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const uint16_t* Kg = static_cast<const uint16_t*>(a.k) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const uint16_t* Vg = static_cast<const uint16_t*>(a.v) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    const uint16_t* Gg = static_cast<const uint16_t*>(a.d_o) + (int64_t)b * T * a.ld_o + (int64_t)h * kD;
    uint16_t* dQg = static_cast<uint16_t*>(a.d_q) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;

    {
        const int qb = qb_own;
        const int qw = qb * kBlk + 32 * wave;  // the wave's first query
        const int q = qw + ln;                 // this lane's query (the products' N index)

        bf16x8 qf[8], gf[8];
        load_frags(qf, Qg, q, T, a.ld_qkv, hh);
        load_frags(gf, Gg, q, T, a.ld_o, hh);
        const float lse2 = q < T ? a.lse2[(int64_t)bh * T + q] : 0.0f;
        const float delta = q < T ? a.delta[(int64_t)bh * T + q] : 0.0f;
        const int lim = a.causal ? min(q, T - 1) : T - 1;  // keys > lim are masked
        floatx16 dq[4];
#pragma unroll
        for (int db = 0; db < 4; ++db) dq[db] = zero16();

        const int k_end = a.causal ? min(qb * kBlk + kBlk, T) : T;
        const int n_steps = (k_end + kTile - 1) / kTile;

        auto dma = [&](DqStage& s, int k0) {
            dma_tile(s.k, Kg, k0, T, a.ld_qkv, voff, wave);
            dma_tile(s.v, Vg, k0, T, a.ld_qkv, voff, wave);
        };
        // kGen: the tile may hold masked keys, or none the wave's queries see
        auto step = [&](auto GEN, const DqStage& s, DqStage& nxt, int k0, bool has_next) __attribute__((always_inline)) {
            constexpr bool kGen = decltype(GEN)::value;
            if (has_next) dma(nxt, k0 + kTile);
            if constexpr (kGen)
                if (a.causal && k0 > qw + 31) return;  // every key of the tile follows the wave's queries
            const bool need_mask = (a.causal && k0 + kTile - 1 > qw) || k0 + kTile > T;
            // masking without branches: element i of key block kb (key k0 + 32*kb + 4*hh + off_i, off_i =
            // 8*(i/4) + i%4 a constant) is masked when off_i > emask[kb], i.e. when key > lim
            int emask[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) emask[kb] = need_mask ? lim - (k0 + 32 * kb + 4 * hh) : INT_MAX;
            // One software-pipelined sequence of 48 bundles (one LDS fragment read three ahead + one MFMA):
            //   bundles  0..15  S^T and dP^T of keys 0..31   (fragment f = b: K / V rows)
            //   bundles 16..31  S^T and dP^T of keys 32..63; dS of keys 0..31, one element per bundle
            //   bundles 32..47  dQ^T += K^T dS^T (fragment f = b: K^T); dS of keys 32..63, two per bundle
            // Row fragment f < 32: 16*kb + 2*cc + w (w = 0: K, 1: V); f >= 32: K^T chunk ci = f - 32 =
            // 8*kb + 4*u + db. Element i of block kb is key k0 + 32*kb + 8*(i/4) + 4*hh + i%4.
            floatx16 sc[2], dp[2];
            float ds[2][16];
            bf16x8 dsb[2][2];
            auto rd = [&](int f) {
                if (f < 32) return read_row((f & 1) ? s.v : s.k, LA.raddr, (f >> 1) & 7, f >> 4);
                return read_tr(s.k, LA.taddr, f - 32);
            };
            auto elem = [&](int kb, int i) {  // dS^T = P^T (dP^T - delta), P^T = exp2(S^T c - lse2)
                float pv = __builtin_amdgcn_exp2f(sc[kb][i] * c - lse2);
                if constexpr (kGen) pv = 8 * (i >> 2) + (i & 3) > emask[kb] ? 0.0f : pv;
                ds[kb][i] = pv * (dp[kb][i] - delta);
            };
            auto pack = [&](int kb, int u) {
                uint32_t wd[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) wd[e] = pack_bf16x2(ds[kb][8 * u + 2 * e], ds[kb][8 * u + 2 * e + 1]);
                dsb[kb][u] = __builtin_bit_cast(bf16x8, make_uint4(wd[0], wd[1], wd[2], wd[3]));
            };
            bf16x8 ring[4];
            ring[0] = rd(0);
            ring[1] = rd(1);
            ring[2] = rd(2);
            static_for<48>([&](auto B) {
                constexpr int b = decltype(B)::value;
                if constexpr (b + 3 < 48) ring[(b + 3) & 3] = rd(b + 3);
                if constexpr (b < 32) {
                    constexpr int kb = b >> 4, cc = (b >> 1) & 7;
                    if constexpr (b & 1) dp[kb] = mfma(ring[b & 3], gf[cc], cc == 0 ? zero16() : dp[kb]);
                    else sc[kb] = mfma(ring[b & 3], qf[cc], cc == 0 ? zero16() : sc[kb]);
                } else {
                    constexpr int ci = b - 32;
                    dq[ci & 3] = mfma(ring[b & 3], dsb[ci >> 3][(ci >> 2) & 1], dq[ci & 3]);
                }
                if constexpr (b >= 16 && b < 32) elem(0, b - 16);
                if constexpr (b == 23 || b == 31) pack(0, b == 31);
                if constexpr (b >= 32 && b < 40) {
                    elem(1, 2 * (b - 32));
                    elem(1, 2 * (b - 32) + 1);
                }
                if constexpr (b == 35 || b == 39) pack(1, b == 39);
                DT_BUNDLE_END;
            });
        };

        // Tiles 0 .. n_plain-1 need no mask (every key at or before the wave's first query and before T); the
        // rest (the diagonal under causality, the tile past T) take the selects and, past the wave's queries,
        // nothing. Two loops, so the first is compiled without them (the same values: emask is INT_MAX).
        const int k_plain = a.causal ? min(qw + 1, T) : T;
        const int n_plain = min(max(k_plain, 0) / kTile, n_steps);
        using True_ = std::true_type;
        using False_ = std::false_type;
        dma(st0, 0);
        stage_barrier();
        int it = 0;
        for (; it + 1 < n_plain; it += 2) {
            const int k0 = it * kTile;
            step(False_{}, st0, st1, k0, it + 1 < n_steps);
            stage_barrier();
            step(False_{}, st1, st0, k0 + kTile, it + 2 < n_steps);
            stage_barrier();
        }
        if (it < n_plain) {  // an odd count: the last plain tile is an even one
            step(False_{}, st0, st1, it * kTile, it + 1 < n_steps);
            stage_barrier();
            ++it;
        }
        for (; it < n_steps; ++it) {
            if (it & 1) step(True_{}, st1, st0, it * kTile, it + 1 < n_steps);
            else step(True_{}, st0, st1, it * kTile, it + 1 < n_steps);
            stage_barrier();
        }
        if (q < T) store_rows(dQg, q, a.ld_grad, hh, dq, a.scale);
    }
}

// ------------------------------------------------------------------------------------------------ dQ from dS
// Eight waves per workgroup share each 64-key tile: wave w takes the block's queries 32*(w & 3) .. +31 and
// dims 64*(w >> 2) .. +63, so every dQ element has one owner and the tiles' products add in key order. The
// tiles stream through a five-stage LDS ring (all 160 KB), four tiles ahead of the one in use (the dS rows
// come from HBM: one tile of lookahead left the kernel waiting on memory latency). One workgroup per CU,
// blocks in decreasing causal cost.
constexpr int kDqThreads = 512;
constexpr int kDqStages = 5;

// LDS stage: a 64-key tile of K and the dS rows of those keys for the block's two 64-query tiles
struct DsqStage {
    uint8_t k[kTileBytes];
    uint8_t ds[2][kDsHalfBytes];
};

// the stage of tile s + 1 has landed (this wave's requests for the three tiles after it, twelve
// instructions, may still be in flight) and every wave is done with the stage of tile s
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// dQ of query block qb_own of (batch, head) bh from the dS the dK/dV pass stored: per 64-key tile a wave
// accumulates its 64 dims of dQ^T += K^T dS^T for its 32 queries (8 MFMAs), K^T and dS^T by transposing reads.
__device__ __forceinline__ void dq_ds_block(const FlashBwdArgs& a, int qb_own, int bh, DsqStage (&st)[kDqStages]) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = wave & 3, dsel = wave >> 2;
    const int ln = lane & 31;
    const int hh = lane >> 5;
    const int T = a.T;
    const int b = bh / a.H, h = bh % a.H;

    // K^T reads of this wave's dim blocks 2*dsel and 2*dsel + 1
    const LaneAddr LA = lane_addr(lane);
    uint32_t taddr[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int d = 0; d < 2; ++d) taddr[r][d] = dsel ? LA.taddr[r][2 + d] : LA.taddr[r][d];
    // K DMA: instruction i of wave w fills rows 32*i + 4*w + lane/16 at chunk position lane%16, fetching the
    // global chunk the swizzle puts there (swz of those rows is 4*(lane/16) + (w & 3))
    uint32_t voff[2];
    {
        const int rlo = lane >> 4;
        const int chunk = (lane & 15) ^ (4 * rlo + (wave & 3));
#pragma unroll
        for (int i = 0; i < 2; ++i) voff[i] = (uint32_t)(((32 * i + 4 * wave + rlo) * a.ld_qkv + 8 * chunk) * 2);
    }
    const uint16_t* Kg = static_cast<const uint16_t*>(a.k) + (int64_t)b * T * a.ld_qkv + (int64_t)h * kD;
    uint16_t* dQg = static_cast<uint16_t*>(a.d_q) + (int64_t)b * T * a.ld_grad + (int64_t)h * kD;
    const BwdDsLayout lay(T, a.causal);
    const uint8_t* ds_head = static_cast<const uint8_t*>(a.ds_ws) + (uint64_t)(bh * lay.per_head()) * kDsBlockBytes;

    const int qw = qb_own * kBlk + 32 * wq;  // the wave's first query
    const int q = qw + ln;
    const int qt = wq >> 1, qh = wq & 1;      // the wave's 64-query tile in the block, its 32-query half there
    // dS^T fragment reads: lane i of 16-lane group G reads key row 4*hh + i/4 (+8 for the second read) of a
    // 16-key chunk, queries 32*qh + 16*(G & 1) + 4*(i & 3) .. +3 (chunk 4*qh + 2*(G & 1) + (i & 1), half
    // (i & 3) / 2, the chunk swizzled by the row); the transposing read hands lane i query 16*(G & 1) + i.
    const int i16 = lane & 15, G = lane >> 4;
    const uint32_t ds_addr = (uint32_t)(qt * kDsHalfBytes + (4 * hh + (i16 >> 2)) * kDsRowBytes +
                                        (((4 * qh + 2 * (G & 1) + (i16 & 1)) ^ (2 * (i16 >> 2))) << 4) + 8 * ((i16 & 3) >> 1));

    floatx16 dq[2] = {zero16(), zero16()};
    const int k_end = a.causal ? min(qb_own * kBlk + kBlk, T) : T;
    const int n_tiles = (k_end + kTile - 1) / kTile;
    const int qt0 = 2 * qb_own;  // the block's first 64-query tile
    const int n_qt = min(2, lay.nqt - qt0);
    // the tiles this wave multiplies: 0 .. n_use-1 (no query of the wave, or every key of a later tile
    // after its queries under causality, leaves the rest to the other waves)
    const int n_use = qw >= T ? 0 : (a.causal ? min(n_tiles, (qw + 31) / kTile + 1) : n_tiles);

    // tile kt -> stage kt % 5: four DMA instructions per wave, also for kt past the range (an empty buffer
    // then: nothing is read, the stage is not used), so that the count of requests in flight is fixed
    // the global unit that LDS chunk wave*64 + lane of a tile's half holds: row 8*wave + lane/8 of the tile
    // (rows of the workspace block: 64*(kt & 1) + that), position lane%8, unit (position) ^ 2*(row & 3)
    uint32_t ds_src;
    {
        const int rl = lane >> 3;
        const int k8 = (lane & 7) ^ (2 * (rl & 3));
        ds_src = (uint32_t)(((((wave >> 2) * 8 + 2 * (wave & 3) + (rl >> 2)) * 32 + (k8 >> 1) * 8 + (rl & 3) * 2 + (k8 & 1)) * 16));
    }
    const uint32_t lds0 = lds_addr(&st[0]);  // stage s starts at lds0 + s * sizeof(DsqStage)
    auto dma = [&](int kt, int stage) {
        const uint32_t sb = lds0 + (uint32_t)stage * (uint32_t)sizeof(DsqStage);
        const bool live = kt < n_tiles;
        const int k0 = live ? kt * kTile : 0;
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(Kg + (int64_t)k0 * a.ld_qkv, live ? (uint32_t)(T - k0) * (uint32_t)a.ld_qkv * 2u : 0u);
        const uint32_t lk = sb + (uint32_t)offsetof(DsqStage, k) + (uint32_t)wave * 1024u;
        dma16(lk, voff[0], rk);
        dma16(lk + 8192, voff[1], rk);
        const int kb = k0 / kBlk;
        const uint8_t* blk = ds_head + (uint64_t)(lay.block_offset(kb) + (qt0 - lay.first_tile(kb))) * kDsBlockBytes;
        const __amdgpu_buffer_rsrc_t r = make_rsrc(blk, live ? (uint32_t)n_qt * kDsBlockBytes : 0u);
        const uint32_t rows = (uint32_t)(kt & 1) * kDsHalfBytes;  // this tile's rows of the key block
        const uint32_t ld = sb + (uint32_t)offsetof(DsqStage, ds) + (uint32_t)wave * 1024u;  // 16-byte chunks wave*64 ..
#pragma unroll
        for (int t = 0; t < 2; ++t) dma16(ld + (uint32_t)t * kDsHalfBytes, (uint32_t)t * kDsBlockBytes + rows + ds_src, r);
    };
    // one tile's product from stage `stage`: the stage's base is added to this lane's five read offsets once,
    // and the reads' remaining offsets are constants (immediate offsets of the LDS reads)
    auto step = [&](int kt, int stage) {
        const uint32_t sb = lds0 + (uint32_t)stage * (uint32_t)sizeof(DsqStage);
        uint32_t kbase[2][2];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int d = 0; d < 2; ++d) kbase[r][d] = taddr[r][d] + sb + (uint32_t)offsetof(DsqStage, k);
        const uint32_t dbase = ds_addr + sb + (uint32_t)offsetof(DsqStage, ds);
        auto tr = [](uint32_t x) { return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(uintptr_t)x); };
        auto read_ds = [&](int c) {  // keys 16*c + {4*hh .. +3, 8 + 4*hh .. +3}: the B operand
            const shortx4 lo = tr(dbase + 16 * c * kDsRowBytes);
            const shortx4 hi = tr(dbase + (16 * c + 8) * kDsRowBytes);
            return __builtin_bit_cast(bf16x8, (shortx8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
        };
        auto read_kt = [&](int c, int d) {  // K^T chunk: keys of 16-key chunk c, dims 32*(2*dsel + d) ..
            const uint32_t rows = (c >> 1) * 8192 + (c & 1) * 4096;
            const shortx4 lo = tr(kbase[0][d] + rows);
            const shortx4 hi = tr(kbase[1][d] + rows + 2048);
            return __builtin_bit_cast(bf16x8, (shortx8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
        };
        // the second 32 keys are all after the wave's queries under causality: their dS was not stored
        const bool second = !a.causal || kt * kTile + 32 <= qw + 31;
        bf16x8 dsf[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) dsf[c] = read_ds(c);
        if (!second) {
            dsf[2] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
            dsf[3] = dsf[2];
        }
        bf16x8 ring[4];
        ring[0] = read_kt(0, 0);
        ring[1] = read_kt(0, 1);
        ring[2] = read_kt(1, 0);
        static_for<8>([&](auto J) {
            constexpr int j = decltype(J)::value;  // chunk j / 2, dim block 2*dsel + j % 2
            if constexpr (j + 3 < 8) ring[(j + 3) & 3] = read_kt((j + 3) >> 1, (j + 3) & 1);
            dq[j & 1] = mfma(ring[j & 3], dsf[j >> 1], dq[j & 1]);
            DT_BUNDLE_END;
        });
    };

    dma(0, 0);
    dma(1, 1);
    dma(2, 2);
    dma(3, 3);
    ring_barrier();  // tile 0 has landed
    // tile kt is in stage s = kt % 5; the request for tile kt + 4 goes to the stage of tile kt - 1, which
    // every wave has finished. A wave's tiles 0 .. n_use-1 and the rest (requests and barriers only) are
    // two loops: a product skipped inside one loop made the compiler copy the accumulators every tile.
    int kt = 0, s = 0;
    for (; kt < n_use; ++kt) {
        dma(kt + 4, s == 0 ? kDqStages - 1 : s - 1);
        step(kt, s);
        ring_barrier();
        s = s == kDqStages - 1 ? 0 : s + 1;
    }
    for (; kt < n_tiles; ++kt) {
        dma(kt + 4, s == 0 ? kDqStages - 1 : s - 1);
        ring_barrier();
        s = s == kDqStages - 1 ? 0 : s + 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the requests past the range, before the workgroup ends
    if (q < T) {
        uint16_t* p = dQg + (int64_t)q * a.ld_grad + 64 * dsel;
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                uint2 w;
                w.x = pack_bf16x2(dq[d][4 * g] * a.scale, dq[d][4 * g + 1] * a.scale);
                w.y = pack_bf16x2(dq[d][4 * g + 2] * a.scale, dq[d][4 * g + 3] * a.scale);
                *reinterpret_cast<uint2*>(p + 32 * d + 8 * g + 4 * hh) = w;
            }
    }
}

// One 128-row block per workgroup, listed in decreasing causal cost, so that the hardware, which hands
// the next workgroup to the first CU that frees up, runs a longest-first schedule.
// pass = 0 (dK/dV) or 1 (dQ): one pass per launch; workgroup BH*j + bh takes, for (batch, head) bh,
//   key block j (dK/dV; key block 0 sees every query tile) or query block n-1-j (dQ).
// pass = 2: both passes in one launch; workgroup 2*BH*j + BH*kind + bh takes the dK/dV of key block j
//   (kind 0) or the dQ of query block n-1-j (kind 1). Under causality both see the same number of 64-row
//   tiles, 2*(n - j) when T is a multiple of 128, so the list is still in decreasing cost (a dK/dV tile,
//   four products, before a dQ tile, three). With at most one block per pass for each CU (T = 2048,
//   B*H = 16) the passes then share the CUs instead of running one after the other, each with its
//   longest block setting its time.
union BwdLds {
    struct {
        DkdvStage s0, s1;
    } kv;
    struct {
        DqStage s0, s1;
    } q;
};

__global__ __launch_bounds__(kThreads, 1) void flash_bwd_bf16_kernel(FlashBwdArgs a, int pass) {
    __shared__ __attribute__((aligned(1024))) BwdLds lds;
    const int BH = a.B * a.H;
    const int n = (a.T + kBlk - 1) / kBlk;
    const int j = (int)blockIdx.x / (pass == 2 ? 2 * BH : BH);
    const int kind = pass == 2 ? ((int)blockIdx.x / BH) & 1 : pass;
    const int bh = (int)blockIdx.x % BH;
    if (kind == 0) dkdv_block<false>(a, j, bh, lds.kv.s0, lds.kv.s1);
    else dq_block(a, n - 1 - j, bh, lds.q.s0, lds.q.s1);
}

// The dS path: the dK/dV pass (workgroup BH*j + bh: key block j) storing dS, then dQ = dS K (workgroup
// BH*j + bh: query block n-1-j), both in decreasing causal cost.
__global__ __launch_bounds__(kThreads, 1) void flash_bwd_dkdv_ds_bf16_kernel(FlashBwdArgs a) {
    __shared__ __attribute__((aligned(1024))) DkdvStage s0, s1;
    const int BH = a.B * a.H;
    dkdv_block<true>(a, (int)blockIdx.x / BH, (int)blockIdx.x % BH, s0, s1);
}
__global__ __launch_bounds__(kDqThreads, 1) void flash_bwd_dq_ds_bf16_kernel(FlashBwdArgs a) {
    __shared__ __attribute__((aligned(1024))) DsqStage st[kDqStages];
    const int BH = a.B * a.H;
    const int n = (a.T + kBlk - 1) / kBlk;
    dq_ds_block(a, n - 1 - (int)blockIdx.x / BH, (int)blockIdx.x % BH, st);
}

}  // namespace

int launch_flash_bwd_bf16(const FlashBwdArgs& a, hipStream_t stream) {
    if ((int64_t)a.T * a.ld_qkv * 2 >= ((int64_t)1 << 31) || (int64_t)a.T * a.ld_o * 2 >= ((int64_t)1 << 31))
        return set_error(DT_ERR_UNSUPPORTED, "extent of one sequence exceeds 2 GiB");
    DT_TRY(launch_flash_bwd_prep(a, 1, stream));
    const int64_t blocks = (int64_t)((a.T + kBlk - 1) / kBlk) * a.B * a.H;  // per pass, one per workgroup
    if (2 * blocks > 0x7fffffff) return set_error(DT_ERR_UNSUPPORTED, "too many workgroups");
    if (a.ds_ws) {  // dS stored by the dK/dV pass, dQ = dS K
        hipLaunchKernelGGL(flash_bwd_dkdv_ds_bf16_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
        DT_HIP_TRY(hipGetLastError());
        hipLaunchKernelGGL(flash_bwd_dq_ds_bf16_kernel, dim3((unsigned)blocks), dim3(kDqThreads), 0, stream, a);
        DT_HIP_TRY(hipGetLastError());
        return DT_OK;
    }
    int cus = 0;
    DT_TRY(persistent_grid(0x7fffffff, &cus));
    if (blocks <= cus) {  // the passes share one launch (measured: T = 2048, B*H = 16: 148 -> 94 us; at
                          // T = 4096, two blocks per CU and pass, one launch per pass is 4 % faster)
        hipLaunchKernelGGL(flash_bwd_bf16_kernel, dim3((unsigned)(2 * blocks)), dim3(kThreads), 0, stream, a, 2);
        DT_HIP_TRY(hipGetLastError());
    } else {
        for (int pass = 0; pass < 2; ++pass) {
            hipLaunchKernelGGL(flash_bwd_bf16_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a, pass);
            DT_HIP_TRY(hipGetLastError());
        }
    }
    return DT_OK;
}

}  // namespace dt
