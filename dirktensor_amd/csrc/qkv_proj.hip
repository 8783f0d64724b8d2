// Fused QKV projection with the q/k RMSNorm + RoPE epilogue, for gfx950 (CDNA4).
//
// Replaces, for the attention layer's input rows x [rows][d_model], the three projections
// q = x Wq^T, k = x Wk^T, v = x Wv^T (OlmoAttention.cpp:68,74,80), q_norm / k_norm over all d_model
// features (:70,:76; RMSNorm.cpp:15-22) and apply_rope on q and k (:84-85, :111-146) with one launch
// that writes rope(norm(q)) | rope(norm(k)) | v into the attention core's input layout
// [rows][3*d_model] (head h of q at columns 128h .. 128h+127).
//
// Work decomposition
//   * A tile is 128 rows x 128 output columns, i.e. one head of q, k or v for 128 token rows, so the
//     rotate-half pairs (d, d+64) of RoPE lie inside a tile. Tiles are numbered row block by row
//     block (q heads, then k heads, then v heads); a persistent grid of G workgroups (a multiple of H,
//     one per CU) takes tile w, w+G, ... With G a multiple of 8 and 3H a multiple of 8, workgroup w
//     runs on XCD w mod 8 and every tile of a column block runs on one XCD, so each block of W passes
//     through one L2.
//   * 8 waves share every k-tile: wave (wr, wc) = (w / 2, w % 2) computes rows 32wr..+32 and columns
//     64wc..+64 of the tile as 1 x 2 blocks of v_mfma_f32_32x32x16_bf16 (fp32 exact mode:
//     v_mfma_f32_32x32x2f32), A = rows of x, B = rows of W, both read along K; every output element
//     has one owner.
//   * The k-tiles (128 bytes of K per row: 64 bf16 or 32 fp32; 32 KB per k-tile for x and W) move from
//     HBM into LDS with buffer_load ... lds through a five-stage ring (all 160 KB), four k-tiles ahead of
//     the one in use: with one k-tile of lookahead a workgroup waited on memory latency. A wave's 4 DMA
//     instructions per k-tile are spread over the current step's MFMAs; past the last k-tile they go out
//     with empty descriptors (nothing is read), so the count of requests in flight is fixed. The
//     descriptors of x end at the last valid row, so rows past it arrive as zeros. LDS rows are 128
//     bytes, the 16-byte chunk c of row r stored at position c ^ ((r >> 1) & 7), so the 16 rows a
//     fragment read touches per cycle hit distinct banks.
//
// Epilogue of a tile: the fp32 tile goes to LDS; each thread then owns 16 columns and
// their rotate-half partners (d, d+64) of one row. A q or k tile computes its rows' sums of squares
// over the head's 128 columns and publishes them; the H tiles of the same row block and tensor run in
// the same round on different workgroups (the grid is at most one workgroup per CU, so every workgroup is
// resident at once). Each published sum is one 64-bit word tagged with the launch's epoch (a number the
// host changes every launch), so a reader polls the H words of its row until all carry this epoch: no
// counters, no fences. The row's sum is then added in a fixed order and
// rms = sqrt(sum / d_model + eps), y = (x / rms) * w, out[d] = y[d] cos - y[d+64] sin,
// out[d+64] = y[d+64] cos + y[d] sin, the reference's rounding order. The words are written and read with
// device-scope coherent accesses (they cross XCDs). A wait that does not end within a bounded spin (about
// a second: a workgroup kept from its CU that long, e.g. by another persistent kernel occupying CUs)
// gives up and writes NaN rows instead of hanging.

#include "dt_internal.h"

#include <type_traits>
#include <utility>

namespace dt {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef unsigned v2u32 __attribute__((ext_vector_type(2)));

constexpr int kTile = 128;               // rows and columns of a work tile
constexpr int kThreads = 512;            // 8 waves
constexpr int kRowB = 128;               // bytes of K per LDS row of a k-tile
constexpr int kOpBytes = kTile * kRowB;  // 16 KB: one operand's k-tile
constexpr int kStages = 5;               // LDS ring of k-tiles (x and W), four ahead of the one in use
constexpr int kStageBytes = 2 * kOpBytes;
constexpr int kRStride = 132;            // floats per row of the fp32 tile in the epilogue
constexpr int kLdsBytes = kStages * kStageBytes;  // 160 KB
static_assert(kLdsBytes >= kTile * kRStride * 4, "the stages must hold the epilogue tile");
constexpr int kBufferDword3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)
constexpr int kCoherent = 16;              // cache policy sc1: device-scope coherent access

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 r = __builtin_convertvector((floatx2){lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferDword3);
}

template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}
#define DT_BUNDLE_END __builtin_amdgcn_sched_barrier(0)

// This wave's LDS DMA and LDS reads are complete before any wave passes it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// The ring's barrier: the k-tile after the one just used has landed (this wave's requests for the three after
// it, twelve instructions, may still be in flight) and every wave is done reading the stage just used.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint4 lds_read16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }

// LDS DMA issued through inline assembly: the compiler does not track these loads, so it does not wait for
// them before reading the other LDS stage (it cannot prove the stages apart, and with the builtin it waits for
// the DMA just issued before the step's first fragment read); the stage barriers wait for them explicitly.
// M0 holds the wave-uniform LDS destination (an operand bound to M0); lane i writes 16 bytes at M0 + 16i.
// s_nop 4 supplies the wait states the hardware needs after an SGPR or M0 write, which the compiler cannot
// see inside the asm.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void dma16(uint32_t lds, uint32_t voff, __amdgpu_buffer_rsrc_t r) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds) : "memory");
}

// One k-tile (128 bytes of K) for one wave: acc[j] += A B_j^T over the tile, A = rows ln of the wave's 32-row
// x band, B_j = rows 32j + ln of its 64-row W band. The 16-byte chunk kk of a row pair (2kk + hh) feeds one
// bf16 MFMA (k 16) or four fp32 MFMAs (k 2 each; lanes hh = 0 and 1 hold k 8kk + e and 8kk + 4 + e).
// Fragments go through a three-deep ring of chunks: bundle (kk, j) reads fragment(s) of chunk kk + 2, so every
// fragment is requested at least three bundles before its MFMA. hook(slot) runs at the start of each of the 8
// bundles (the caller's memory requests, spread over the step).
template <bool kF32, typename Hook>
__device__ __forceinline__ void tile_step(floatx16 (&acc)[2], const uint8_t* As, const uint8_t* Bs,
                                          const uint32_t (&coff)[4], Hook&& hook) {
    uint4 fr[3][3];  // [chunk % 3][a, b0, b1]
    auto rd = [&](int c, int m) { return m == 0 ? lds_read16(As + coff[c]) : lds_read16(Bs + 4096 * (m - 1) + coff[c]); };
#pragma unroll
    for (int m = 0; m < 3; ++m) fr[0][m] = rd(0, m);
#pragma unroll
    for (int m = 0; m < 3; ++m) fr[1][m] = rd(1, m);
    static_for<4>([&](auto KK) {
        constexpr int kk = decltype(KK)::value;
        static_for<2>([&](auto J) {
            constexpr int j = decltype(J)::value;
            hook(std::integral_constant<int, 2 * kk + j>{});
            if constexpr (kk + 2 < 4) {
                if constexpr (j == 0) {
                    fr[(kk + 2) % 3][0] = rd(kk + 2, 0);
                    fr[(kk + 2) % 3][1] = rd(kk + 2, 1);
                } else {
                    fr[(kk + 2) % 3][2] = rd(kk + 2, 2);
                }
            }
            const uint4 fa = fr[kk % 3][0], fb = fr[kk % 3][1 + j];
            if constexpr (kF32) {
                const floatx4 av = __builtin_bit_cast(floatx4, fa);
                const floatx4 bv = __builtin_bit_cast(floatx4, fb);
                static_for<4>([&](auto E) {
                    constexpr int e = decltype(E)::value;
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[e], bv[e], acc[j], 0, 0, 0);
                });
            } else {
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa),
                                                               __builtin_bit_cast(bf16x8, fb), acc[j], 0, 0, 0);
            }
            DT_BUNDLE_END;
        });
    });
}

template <bool kF32>
__device__ __forceinline__ void store4(void* base, int64_t idx, float4 v) {  // 4 values from element idx
    if constexpr (kF32) {
        *reinterpret_cast<float4*>(static_cast<float*>(base) + idx) = v;
    } else {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + idx) = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    }
}

template <bool kF32>
__global__ __launch_bounds__(kThreads, 1) void qkv_norm_rope_kernel(QkvArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kLdsBytes];
    constexpr int es = kF32 ? 4 : 2;  // bytes per element of x, W and the outputs

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave >> 1, wc = wave & 1;  // the wave's 32-row band of x and 64-row band of W
    const int ln = lane & 31, hh = lane >> 5;
    const int H = a.H, dm = H * 128, ncb = 3 * H;
    const int nk = dm * es / kRowB;  // k-tiles
    const int n_tiles = (a.rows + kTile - 1) / kTile * ncb;

    // DMA: instruction i of wave w fills LDS rows 8*(8i + w) .. +8 of an operand's k-tile (1 KB); lane -> row
    // 8*(8i + w) + lane/8 at chunk position lane%8, holding the global chunk (lane%8) ^ ((row >> 1) & 7), where
    // (row >> 1) & 7 = (4*(w & 1) + lane/16) & 7 does not depend on i
    uint32_t offx[2], offw[2];
    {
        const int gc = (lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = 8 * (8 * i + wave) + (lane >> 3);
            offx[i] = (uint32_t)(r * a.ldx * es + 16 * gc);
            offw[i] = (uint32_t)(r * dm * es + 16 * gc);
        }
    }
    // fragment reads: row 32*blk + ln of the wave's band, chunk 2kk + hh at position (2kk + hh) ^ ((ln >> 1) & 7)
    uint32_t coff[4];
    {
        const int f = (ln >> 1) & 7;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) coff[kk] = (uint32_t)((((2 * kk + hh) ^ f)) * 16);
    }
    const uint32_t arow = (uint32_t)((32 * wr + ln) * kRowB);
    const uint32_t brow = (uint32_t)((64 * wc + ln) * kRowB);

    const __amdgpu_buffer_rsrc_t rss = make_rsrc(a.ss, (uint32_t)a.ss_bytes);
    const __amdgpu_buffer_rsrc_t rstat = make_rsrc(a.status, 4u);
    float* const R0 = reinterpret_cast<float*>(lds);

    for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        const int rb = tile / ncb, cb = tile - rb * ncb;
        const int which = cb / H, head = cb - which * H;  // 0 q, 1 k, 2 v
        const int row0 = rb * kTile;
        const int nrows = min(kTile, a.rows - row0);
        const char* xg = static_cast<const char*>(a.x) + (int64_t)row0 * a.ldx * es;
        const char* wg = static_cast<const char*>(a.w) + (int64_t)cb * kTile * dm * es;
        const uint32_t xbytes = (uint32_t)(nrows * a.ldx * es);
        const uint32_t wbytes = (uint32_t)(kTile * dm * es);

        // k-tile kt of x and W -> stage kt % kStages (rows of x past the last arrive as zeros): DMA instruction
        // q (0-1 x, 2-3 W) of this wave; a k-tile past the last gets empty descriptors
        auto dma_one = [&](int kt, auto Q) {
            constexpr int q = decltype(Q)::value;
            const bool live = kt < nk;
            const uint32_t koff = live ? (uint32_t)(kt * kRowB) : 0u;
            const uint32_t l0 = lds_addr(lds + (kt % kStages) * kStageBytes);
            if constexpr (q < 2)
                dma16(l0 + (8 * q + wave) * 1024, offx[q], make_rsrc(xg + koff, live ? xbytes - koff : 0u));
            else
                dma16(l0 + kOpBytes + (8 * (q - 2) + wave) * 1024, offw[q - 2], make_rsrc(wg + koff, live ? wbytes - koff : 0u));
        };
        auto dma = [&](int kt) { static_for<4>([&](auto Q) { dma_one(kt, Q); }); };

        floatx16 acc[2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;

        static_for<kStages - 1>([&](auto K) { dma(decltype(K)::value); });
        ring_barrier();  // k-tile 0 has landed
        // step kt: compute from stage kt % 5 while k-tile kt + 4 goes out into the stage of k-tile kt - 1 (every
        // wave finished it before the last barrier), one DMA instruction before every other bundle
        for (int kt = 0; kt < nk; ++kt) {
            const uint8_t* As = lds + (kt % kStages) * kStageBytes;
            tile_step<kF32>(acc, As + arow, As + kOpBytes + brow, coff, [&](auto SLOT) {
                constexpr int slot = decltype(SLOT)::value;
                if constexpr ((slot & 1) == 0) dma_one(kt + kStages - 1, std::integral_constant<int, slot / 2>{});
            });
            ring_barrier();
        }
        stage_barrier();  // no load in flight (the empty ones included) and no wave reads a stage any more

        // the fp32 tile, row-major: element (j, e) is row 32wr + 8(e/4) + 4hh + e%4, column 64wc + 32j + ln
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                R0[(32 * wr + 8 * (e >> 2) + 4 * hh + (e & 3)) * kRStride + 64 * wc + 32 * j + ln] = acc[j][e];
        __syncthreads();

        // thread -> row er of the tile, columns 16qd .. +16 and their rotate-half partners 64 + 16qd .. +16, read
        // from the tile 4 columns at a time
        const int er = tid >> 2, qd = tid & 3;
        auto cols4 = [&](int c) { return *reinterpret_cast<const float4*>(&R0[er * kRStride + c]); };
        const bool valid = er < nrows;
        const int64_t grow = (int64_t)row0 + er;
        const int64_t ocol = (int64_t)cb * kTile + 16 * qd;  // = which*dm + head*128 + 16qd
        if (which == 2) {  // v: the projection itself
            if (valid) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    store4<kF32>(a.out, grow * a.ld_out + ocol + 4 * k, cols4(16 * qd + 4 * k));
                    store4<kF32>(a.out, grow * a.ld_out + ocol + 64 + 4 * k, cols4(64 + 16 * qd + 4 * k));
                }
            }
        } else {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 u = cols4(16 * qd + 4 * k), v = cols4(64 + 16 * qd + 4 * k);
                ss += u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w + v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                if (a.pre && valid) {  // the pre-norm projection, kept for the norms' backward
                    store4<kF32>(a.pre, grow * a.ld_pre + ocol + 4 * k, u);
                    store4<kF32>(a.pre, grow * a.ld_pre + ocol + 64 + 4 * k, v);
                }
            }
            ss += __shfl_xor(ss, 1, 64);
            ss += __shfl_xor(ss, 2, 64);
            // this head's sum of squares of row grow -> ss[grow][which][head], as one 64-bit word tagged with the
            // launch's epoch (the word is written whole, so a reader sees the old entry or the new one)
            const uint32_t srow = (uint32_t)((grow * 2 + which) * H) * 8u;
            if (qd == 0 && valid) {
                const uint64_t word = ((uint64_t)a.epoch << 32) | __builtin_bit_cast(uint32_t, ss);
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32, word), rss, srow + 8u * head, 0,
                                                      kCoherent);
            }
            if (valid) {
                // the other H - 1 tiles of this row block and tensor run in the same round on other workgroups:
                // thread qd polls heads 4qd .. 4qd+3 of its row until all four carry this launch's epoch
                float part = 0.0f;
                bool ok = false;
                for (int spins = 0; spins < a.spin_limit; ++spins) {
                    bool all = true;
                    float sum = 0.0f;
                    for (int h = 4 * qd; h < H; h += 16) {  // heads 4qd + 16j .. +3: each head once (H % 4 == 0)
                        // (the loaded vectors are bit-cast whole: extracting elements 0 and 2 of the builtin's
                        // result directly makes this compiler narrow the load to one dword and read it twice)
                        const uint4 p0 = __builtin_bit_cast(
                            uint4, __builtin_amdgcn_raw_buffer_load_b128(rss, srow + 8u * h, 0, kCoherent));
                        const uint4 p1 = __builtin_bit_cast(
                            uint4, __builtin_amdgcn_raw_buffer_load_b128(rss, srow + 8u * h + 16u, 0, kCoherent));
                        all = all && p0.y == a.epoch && p0.w == a.epoch && p1.y == a.epoch && p1.w == a.epoch;
                        sum += __builtin_bit_cast(float, p0.x);
                        sum += __builtin_bit_cast(float, p0.z);
                        sum += __builtin_bit_cast(float, p1.x);
                        sum += __builtin_bit_cast(float, p1.z);
                    }
                    if (all) {
                        part = sum;
                        ok = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                // the row's total, added in the same order by its four threads: (q0 + q1) + (q2 + q3)
                part += __shfl_xor(part, 1, 64);
                part += __shfl_xor(part, 2, 64);
                const bool all_ok =
                    __shfl_xor((int)ok, 1, 64) & __shfl_xor((int)ok, 2, 64) & __shfl_xor((int)ok, 3, 64) & (int)ok;
                const float tot = part;
                const float rms = all_ok ? sqrtf(tot / (float)dm + a.eps) : __builtin_nanf("");
                if (!all_ok && qd == 0)  // the host reports it (dt_ctx_check, synchronous host-memory calls)
                    __builtin_amdgcn_raw_buffer_store_b32(kQkvWaitGaveUp, rstat, 0, 0, 0);
                if (a.rms && qd == 0) a.rms[(int64_t)which * a.rows + grow] = rms;
                const int t = (int)(grow % a.T);
                const float* cs = a.rope_cos + (int64_t)t * 64 + 16 * qd;
                const float* sn = a.rope_sin + (int64_t)t * 64 + 16 * qd;
                const float* wn = (which == 0 ? a.q_w : a.k_w) + head * 128 + 16 * qd;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 u = cols4(16 * qd + 4 * k), v = cols4(64 + 16 * qd + 4 * k);
                    const float4 c4 = *reinterpret_cast<const float4*>(cs + 4 * k);
                    const float4 s4 = *reinterpret_cast<const float4*>(sn + 4 * k);
                    const float4 w0 = *reinterpret_cast<const float4*>(wn + 4 * k);
                    const float4 w1 = *reinterpret_cast<const float4*>(wn + 64 + 4 * k);
                    const float uv[4] = {u.x, u.y, u.z, u.w}, vv[4] = {v.x, v.y, v.z, v.w};
                    const float cv[4] = {c4.x, c4.y, c4.z, c4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
                    const float wv0[4] = {w0.x, w0.y, w0.z, w0.w}, wv1[4] = {w1.x, w1.y, w1.z, w1.w};
                    float r0[4], r1[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float y0 = (uv[e] / rms) * wv0[e];
                        const float y1 = (vv[e] / rms) * wv1[e];
                        r0[e] = y0 * cv[e] - y1 * sv[e];
                        r1[e] = y1 * cv[e] + y0 * sv[e];
                    }
                    store4<kF32>(a.out, grow * a.ld_out + ocol + 4 * k, make_float4(r0[0], r0[1], r0[2], r0[3]));
                    store4<kF32>(a.out, grow * a.ld_out + ocol + 64 + 4 * k, make_float4(r1[0], r1[1], r1[2], r1[3]));
                }
            }
        }
        __syncthreads();  // every thread has read the epilogue tiles before the next tile's DMA overwrites them
    }
}

}  // namespace

int qkv_norm_rope_workspace(int rows, int H, size_t* ss_bytes) {
    const int64_t n_rb = ((int64_t)rows + kTile - 1) / kTile;
    *ss_bytes = (size_t)(n_rb * kTile) * 2 * H * sizeof(uint64_t);
    return DT_OK;
}

int qkv_fused_one_round(int rows, int H, bool* fits) {
    int cus = 0;
    DT_TRY(persistent_grid(0x7fffffff, &cus));
    const int64_t n_tiles = ((int64_t)rows + kTile - 1) / kTile * 3 * H;
    *fits = H >= 4 && H % 4 == 0 && n_tiles <= (cus / H) * (int64_t)H;
    return DT_OK;
}

int launch_qkv_norm_rope(const QkvArgs& a, int f32, hipStream_t stream) {
    const int es = f32 ? 4 : 2;
    if (a.H < 4 || a.H % 4 != 0) return set_error(DT_ERR_UNSUPPORTED, "fused QKV: H=%d must be a positive multiple of 4", a.H);
    if (a.rows < 1 || a.T < 1) return set_error(DT_ERR_INVALID_ARG, "fused QKV: rows=%d, T=%d", a.rows, a.T);
    const int64_t dm = (int64_t)a.H * 128;
    if (a.ldx < dm || a.ld_out < 3 * dm || (a.pre && a.ld_pre < 3 * dm))
        return set_error(DT_ERR_INVALID_ARG, "fused QKV: row strides below the row width");
    if ((int64_t)kTile * a.ldx * es >= ((int64_t)1 << 31) || (int64_t)kTile * dm * es >= ((int64_t)1 << 31))
        return set_error(DT_ERR_UNSUPPORTED, "fused QKV: a 128-row band exceeds 2 GiB");
    if (a.epoch == 0) return set_error(DT_ERR_INVALID_ARG, "fused QKV: epoch 0 is reserved");
    if (!a.status || a.spin_limit < 0) return set_error(DT_ERR_INVALID_ARG, "fused QKV: no status word or a negative spin limit");
    size_t ssb = 0;
    DT_TRY(qkv_norm_rope_workspace(a.rows, a.H, &ssb));
    if (ssb >= ((size_t)1 << 31) || a.ss_bytes < (int64_t)ssb)
        return set_error(DT_ERR_UNSUPPORTED, "fused QKV: partial-sum workspace too small or above 2 GiB");
    int cus = 0;
    DT_TRY(persistent_grid(0x7fffffff, &cus));
    const int64_t n_tiles = ((int64_t)a.rows + kTile - 1) / kTile * 3 * a.H;
    if (n_tiles > 0x7fffffff) return set_error(DT_ERR_UNSUPPORTED, "fused QKV: too many tiles");
    // at most one workgroup per CU (its LDS use admits no second one), so all of them are resident together;
    // a multiple of H, so the H tiles of a row block and tensor always fall in one round (with H a multiple of
    // 8, as at the OLMo-2 shapes, also a multiple of 8: the column-block -> XCD mapping holds)
    int64_t g = (cus / a.H) * (int64_t)a.H;
    if (g < a.H) return set_error(DT_ERR_UNSUPPORTED, "fused QKV: H=%d exceeds the %d CUs", a.H, cus);
    if (g > n_tiles) g = n_tiles;
    if (f32) hipLaunchKernelGGL(qkv_norm_rope_kernel<true>, dim3((unsigned)g), dim3(kThreads), 0, stream, a);
    else hipLaunchKernelGGL(qkv_norm_rope_kernel<false>, dim3((unsigned)g), dim3(kThreads), 0, stream, a);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
