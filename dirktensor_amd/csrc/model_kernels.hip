// Element-wise and row kernels of the OLMo-2 model around the attention layer, for gfx950.
//
//   embed_gather        OlmoModel.cpp:29-38: x[b, t] = E[token[b, t]]
//   rmsnorm_rows        RMSNorm::forward (RMSNorm.cpp:15-22) on d_model rows, optionally added to a
//                       residual (the post-norm blocks, OlmoBlock.cpp:13-21: h = x + N(attn(x))),
//                       keeping the output y and rms the norm's backward needs (RMSNorm.h:22-23)
//   swiglu              OlmoMlp.cpp:44-53: act = gate / (1 + exp(-gate)) * up, from the [gate | up]
//                       rows of the concatenated projection
//   ce_rows / ce_reduce ce_loss (CrossEntropyLoss.cpp:8-43) and the gradient main.cpp:62-80 builds
//   rmsnorm_bwd_rows    RMSNorm::backward (RMSNorm.cpp:24-36) with the weight gradient reduced
//                       deterministically through per-workgroup partial sums
//   swiglu_bwd          OlmoMlp.cpp (backward): d_up = d_act * silu(gate),
//                       d_gate = d_act * up * sig * (1 + gate * (1 - sig))
//   embed_bwd           OlmoModel.cpp:57-66: E_grad[token] += dx rows, summed per distinct token in
//                       position order (no atomics)
// All are HBM bound; one workgroup of 256 threads per row unless noted.

#include "dt_internal.h"

namespace dt {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 r = __builtin_convertvector((floatx2){lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, r);
}

// sum over the 256 threads of a workgroup (4 waves)
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    __syncthreads();  // red may still be read by a previous call
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void embed_gather_kernel(const int32_t* tok, const float* E, float* x, int dm) {
    const int64_t row = blockIdx.x;
    const float4* src = reinterpret_cast<const float4*>(E + (int64_t)tok[row] * dm);
    float4* dst = reinterpret_cast<float4*>(x + row * dm);
    for (int i = threadIdx.x; i < dm / 4; i += 256) dst[i] = src[i];
}

// The same for rows of dm = 1024 * kChunks: the row stays in registers (kChunks float4 per thread) between the
// sum of squares and the output pass instead of being read a second time.
template <int kChunks>
__global__ __launch_bounds__(256) void rmsnorm_rows_reg_kernel(const float* a, const float* w, const float* res,
                                                               float* out, uint16_t* out16, float* y_save,
                                                               float* rms_save, int dm, float eps) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const float* ar = a + row * dm;
    float4 v[kChunks];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        v[c] = *reinterpret_cast<const float4*>(ar + 4 * threadIdx.x + 1024 * c);
        ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
    }
    ss = block_sum(ss, red);
    const float rms = sqrtf(ss / (float)dm + eps);
    if (rms_save && threadIdx.x == 0) rms_save[row] = rms;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int i = 4 * threadIdx.x + 1024 * c;
        const float4 wv = *reinterpret_cast<const float4*>(w + i);
        const float4 y = make_float4((v[c].x / rms) * wv.x, (v[c].y / rms) * wv.y, (v[c].z / rms) * wv.z,
                                     (v[c].w / rms) * wv.w);
        if (y_save) *reinterpret_cast<float4*>(y_save + row * dm + i) = y;
        float4 o = y;
        if (res) {
            const float4 r = *reinterpret_cast<const float4*>(res + row * dm + i);
            o = make_float4(r.x + y.x, r.y + y.y, r.z + y.z, r.w + y.w);
        }
        *reinterpret_cast<float4*>(out + row * dm + i) = o;
        if (out16) {
            uint2 p;
            p.x = pack_bf16x2(o.x, o.y);
            p.y = pack_bf16x2(o.z, o.w);
            *reinterpret_cast<uint2*>(out16 + row * dm + i) = p;
        }
    }
}

// out = res + (a / rms) * w (res may be null); y_save = (a / rms) * w, rms_save = rms (either may be null);
// out16 (nullable) receives a bf16 copy of out
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* a, const float* w, const float* res, float* out,
                                                           uint16_t* out16, float* y_save, float* rms_save, int dm,
                                                           float eps) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const float* ar = a + row * dm;
    float ss = 0.0f;
    for (int i = 4 * threadIdx.x; i < dm; i += 1024) {
        const float4 v = *reinterpret_cast<const float4*>(ar + i);
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = block_sum(ss, red);
    const float rms = sqrtf(ss / (float)dm + eps);
    if (rms_save && threadIdx.x == 0) rms_save[row] = rms;
    for (int i = 4 * threadIdx.x; i < dm; i += 1024) {
        const float4 v = *reinterpret_cast<const float4*>(ar + i);
        const float4 wv = *reinterpret_cast<const float4*>(w + i);
        const float4 y = make_float4((v.x / rms) * wv.x, (v.y / rms) * wv.y, (v.z / rms) * wv.z, (v.w / rms) * wv.w);
        if (y_save) *reinterpret_cast<float4*>(y_save + row * dm + i) = y;
        float4 o = y;
        if (res) {
            const float4 r = *reinterpret_cast<const float4*>(res + row * dm + i);
            o = make_float4(r.x + y.x, r.y + y.y, r.z + y.z, r.w + y.w);
        }
        *reinterpret_cast<float4*>(out + row * dm + i) = o;
        if (out16) {
            uint2 p;
            p.x = pack_bf16x2(o.x, o.y);
            p.y = pack_bf16x2(o.z, o.w);
            *reinterpret_cast<uint2*>(out16 + row * dm + i) = p;
        }
    }
}

__device__ __forceinline__ float4 load4(const void* p, int64_t idx, bool bf16) {
    if (bf16) {
        const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + idx);
        return make_float4(__builtin_bit_cast(float, w.x << 16), __builtin_bit_cast(float, w.x & 0xffff0000u),
                           __builtin_bit_cast(float, w.y << 16), __builtin_bit_cast(float, w.y & 0xffff0000u));
    }
    return *reinterpret_cast<const float4*>(static_cast<const float*>(p) + idx);
}
__device__ __forceinline__ float load1(const void* p, int64_t idx, bool bf16) {
    if (bf16) return __builtin_bit_cast(float, (uint32_t)static_cast<const uint16_t*>(p)[idx] << 16);
    return static_cast<const float*>(p)[idx];
}

// act[r][i] = silu(gu[r][i]) * gu[r][hid + i]; gu and act both fp32, or both bf16 (grid-stride over rows * hid / 4)
template <bool kBF16>
__global__ __launch_bounds__(256) void swiglu_kernel(const void* gu, void* act, int64_t rows, int hid) {
    const int64_t n4 = rows * (hid / 4);
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < n4; q += (int64_t)gridDim.x * 256) {
        const int64_t r = q / (hid / 4);
        const int i = (int)(q - r * (hid / 4)) * 4;
        const float4 g = load4(gu, r * 2 * hid + i, kBF16);
        const float4 u = load4(gu, r * 2 * hid + hid + i, kBF16);
        const float4 o = make_float4(g.x / (1.0f + expf(-g.x)) * u.x, g.y / (1.0f + expf(-g.y)) * u.y,
                                     g.z / (1.0f + expf(-g.z)) * u.z, g.w / (1.0f + expf(-g.w)) * u.w);
        if constexpr (kBF16) {
            uint2 p;
            p.x = pack_bf16x2(o.x, o.y);
            p.y = pack_bf16x2(o.z, o.w);
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(act) + r * hid + i) = p;
        } else {
            *reinterpret_cast<float4*>(static_cast<float*>(act) + r * hid + i) = o;
        }
    }
}

// bf16 [gate | up] -> bf16 act, eight elements (16 bytes) per thread and step (hid % 8 == 0)
__global__ __launch_bounds__(256) void swiglu_bf16x8_kernel(const uint16_t* gu, uint16_t* act, int64_t rows, int hid) {
    const int64_t n8 = rows * (hid / 8);
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < n8; q += (int64_t)gridDim.x * 256) {
        const int64_t r = q / (hid / 8);
        const int i = (int)(q - r * (hid / 8)) * 8;
        const uint4 g = *reinterpret_cast<const uint4*>(gu + r * 2 * hid + i);
        const uint4 u = *reinterpret_cast<const uint4*>(gu + r * 2 * hid + hid + i);
        const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
        uint32_t ow[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float g0 = __builtin_bit_cast(float, gw[e] << 16), g1 = __builtin_bit_cast(float, gw[e] & 0xffff0000u);
            const float u0 = __builtin_bit_cast(float, uw[e] << 16), u1 = __builtin_bit_cast(float, uw[e] & 0xffff0000u);
            ow[e] = pack_bf16x2(g0 / (1.0f + expf(-g0)) * u0, g1 / (1.0f + expf(-g1)) * u1);
        }
        *reinterpret_cast<uint4*>(act + r * hid + i) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
}

// One row of logits: target[row] >= 0 is the next token (a loss term), -1 none (no loss, zero gradient).
// term[row] = log(sum exp(l - max)) - (l[target] - max); grad row (nullable) = (softmax - onehot) * inv_count.
// inv_count is NaN when no position has a target: the reference then divides by zero (CrossEntropyLoss.cpp:40,
// main.cpp:88), so the loss and every gradient element are NaN, the rows without a target included.
// grad may alias logits (main.cpp turns probs into the gradient in place): every element is read and then
// written by the same thread, and l[target] is read before any thread writes.
// kVec4: V % 4 == 0 and 16-byte aligned rows, read and written as float4 (HBM bound: two reads of the row
// and one write of the gradient).
template <bool kVec4>
__global__ __launch_bounds__(256) void ce_rows_kernel(const float* logits, const int32_t* target, float* term,
                                                      float* grad, int V, float inv_count) {
    __shared__ float red_m[4], red_s[4];
    const int64_t row = blockIdx.x;
    const int tgt = target[row];
    const float* l = logits + row * V;
    float* g = grad ? grad + row * V : nullptr;
    if (tgt < 0) {
        if (threadIdx.x == 0) term[row] = 0.0f;
        if (g)
            for (int i = threadIdx.x; i < V; i += 256) g[i] = 0.0f * inv_count;
        return;
    }
    const float l_tgt = threadIdx.x == 0 ? l[tgt] : 0.0f;  // before the barrier: the gradient may overwrite it
    // online (max, sum of exp) per thread, then combined over the workgroup
    float m = -__builtin_huge_valf(), s = 0.0f;
    if constexpr (kVec4) {
        for (int i = threadIdx.x; i < V / 4; i += 256) {
            const float4 x = reinterpret_cast<const float4*>(l)[i];
            const float xm = fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w));
            if (xm > m) {
                s = s * expf(m - xm);
                m = xm;
            }
            s += (expf(x.x - m) + expf(x.y - m)) + (expf(x.z - m) + expf(x.w - m));
        }
    } else {
        for (int i = threadIdx.x; i < V; i += 256) {
            const float x = l[i];
            if (x > m) {
                s = s * expf(m - x) + 1.0f;
                m = x;
            } else {
                s += expf(x - m);
            }
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float m2 = __shfl_xor(m, off, 64), s2 = __shfl_xor(s, off, 64);
        const float mm = fmaxf(m, m2);
        s = (m == -__builtin_huge_valf() ? 0.0f : s * expf(m - mm)) + (m2 == -__builtin_huge_valf() ? 0.0f : s2 * expf(m2 - mm));
        m = mm;
    }
    if ((threadIdx.x & 63) == 0) {
        red_m[threadIdx.x >> 6] = m;
        red_s[threadIdx.x >> 6] = s;
    }
    __syncthreads();
    float mx = red_m[0];
    for (int k = 1; k < 4; ++k) mx = fmaxf(mx, red_m[k]);
    float se = 0.0f;
    for (int k = 0; k < 4; ++k) se += red_s[k] * expf(red_m[k] - mx);
    if (threadIdx.x == 0) term[row] = logf(se) - (l_tgt - mx);
    if (g) {
        const float inv = 1.0f / se;
        if constexpr (kVec4) {
            for (int i = threadIdx.x; i < V / 4; i += 256) {
                const float4 x = reinterpret_cast<const float4*>(l)[i];
                float p[4] = {expf(x.x - mx) * inv, expf(x.y - mx) * inv, expf(x.z - mx) * inv, expf(x.w - mx) * inv};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * i + e == tgt) p[e] -= 1.0f;
                reinterpret_cast<float4*>(g)[i] =
                    make_float4(p[0] * inv_count, p[1] * inv_count, p[2] * inv_count, p[3] * inv_count);
            }
        } else {
            for (int i = threadIdx.x; i < V; i += 256) {
                float p = expf(l[i] - mx) * inv;
                if (i == tgt) p -= 1.0f;
                g[i] = p * inv_count;
            }
        }
    }
}

// The same row with the whole row held in registers (kChunks float4 per thread, 1024 threads, so V / 4 <= 1024 *
// kChunks; V % 4 == 0, 16-byte aligned rows): the row is read from memory once instead of twice. The row's
// maximum is formed first and the sum of exponentials then taken relative to it.
template <int kChunks>
__global__ __launch_bounds__(1024) void ce_rows_reg_kernel(const float* logits, const int32_t* target, float* term,
                                                           float* grad, int V, float inv_count) {
    __shared__ float red[16];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int64_t row = blockIdx.x;
    const int tgt = target[row];
    const float* l = logits + row * V;
    float* g = grad ? grad + row * V : nullptr;
    const int V4 = V / 4;
    if (tgt < 0) {
        if (tid == 0) term[row] = 0.0f;
        if (g)
            for (int i = tid; i < V4; i += 1024)
                reinterpret_cast<float4*>(g)[i] = make_float4(0.0f * inv_count, 0.0f * inv_count, 0.0f * inv_count,
                                                              0.0f * inv_count);
        return;
    }
    const float l_tgt = tid == 0 ? l[tgt] : 0.0f;  // before the barriers: the gradient may overwrite it
    constexpr float kNegInf = -__builtin_huge_valf();
    float4 x[kChunks];
    float m = kNegInf;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int i = c * 1024 + tid;
        x[c] = i < V4 ? reinterpret_cast<const float4*>(l)[i] : make_float4(kNegInf, kNegInf, kNegInf, kNegInf);
        m = fmaxf(m, fmaxf(fmaxf(x[c].x, x[c].y), fmaxf(x[c].z, x[c].w)));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) red[wv] = m;
    __syncthreads();
    float mx = red[0];
    for (int k = 1; k < 16; ++k) mx = fmaxf(mx, red[k]);
    __syncthreads();  // red is reused below
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
        s += (expf(x[c].x - mx) + expf(x[c].y - mx)) + (expf(x[c].z - mx) + expf(x[c].w - mx));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) red[wv] = s;
    __syncthreads();
    float se = 0.0f;
    for (int k = 0; k < 16; ++k) se += red[k];
    if (tid == 0) term[row] = logf(se) - (l_tgt - mx);
    if (g) {
        const float inv = 1.0f / se;
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
            const int i = c * 1024 + tid;
            if (i < V4) {
                float p[4] = {expf(x[c].x - mx) * inv, expf(x[c].y - mx) * inv, expf(x[c].z - mx) * inv,
                              expf(x[c].w - mx) * inv};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * i + e == tgt) p[e] -= 1.0f;
                reinterpret_cast<float4*>(g)[i] =
                    make_float4(p[0] * inv_count, p[1] * inv_count, p[2] * inv_count, p[3] * inv_count);
            }
        }
    }
}
constexpr int kCeChunks = 25;  // rows of up to 102400 logits in registers

// loss = sum of the terms (fixed order, fp64) / count, one workgroup
__global__ __launch_bounds__(256) void ce_reduce_kernel(const float* term, int64_t rows, float inv_count, float* loss) {
    __shared__ double red[256];
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < rows; i += 256) acc += term[i];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) loss[0] = (float)(red[0] * (double)inv_count);
}

// RMSNorm::backward for kRowsPerBlock rows per workgroup: c = mean(dy * y), n = y / w,
// dx = (w * dy - n * c) / rms; this workgroup's column sums of dy * n go to partial[blockIdx.x][dm].
// dx_add (nullable) is added to dx (the residual branch of the block's backward, OlmoBlock.cpp:28,32).
constexpr int kRowsPerBlock = 4;  // 512 workgroups for 2048 rows
__global__ __launch_bounds__(256) void rmsnorm_bwd_rows_kernel(const float* dy, const float* y, const float* rms,
                                                               const float* w, const float* dx_add, float* dx,
                                                               uint16_t* dx16, float* partial, int64_t rows, int dm) {
    __shared__ float red[4];
    __shared__ float cs[kRowsPerBlock];
    const int64_t r0 = (int64_t)blockIdx.x * kRowsPerBlock;
    const int nr = (int)min((int64_t)kRowsPerBlock, rows - r0);
    for (int k = 0; k < nr; ++k) {
        const int64_t row = r0 + k;
        float acc = 0.0f;
        for (int i = 4 * threadIdx.x; i < dm; i += 1024) {
            const float4 g = *reinterpret_cast<const float4*>(dy + row * dm + i);
            const float4 v = *reinterpret_cast<const float4*>(y + row * dm + i);
            acc += g.x * v.x + g.y * v.y + g.z * v.z + g.w * v.w;
        }
        acc = block_sum(acc, red);
        if (threadIdx.x == 0) cs[k] = acc / (float)dm;
    }
    __syncthreads();
    for (int i = 4 * threadIdx.x; i < dm; i += 1024) {
        const float4 wv = *reinterpret_cast<const float4*>(w + i);
        float4 p = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int k = 0; k < nr; ++k) {
            const int64_t row = r0 + k;
            const float c = cs[k], inv = 1.0f / rms[row];
            const float4 g = *reinterpret_cast<const float4*>(dy + row * dm + i);
            const float4 v = *reinterpret_cast<const float4*>(y + row * dm + i);
            const float4 n = make_float4(v.x / wv.x, v.y / wv.y, v.z / wv.z, v.w / wv.w);
            float4 o = make_float4((wv.x * g.x - n.x * c) * inv, (wv.y * g.y - n.y * c) * inv,
                                   (wv.z * g.z - n.z * c) * inv, (wv.w * g.w - n.w * c) * inv);
            if (dx_add) {
                const float4 e = *reinterpret_cast<const float4*>(dx_add + row * dm + i);
                o = make_float4(o.x + e.x, o.y + e.y, o.z + e.z, o.w + e.w);
            }
            if (dx) *reinterpret_cast<float4*>(dx + row * dm + i) = o;
            if (dx16) {  // the same values rounded to bf16, as f32_to_bf16 rounds them
                uint2 b;
                b.x = pack_bf16x2(o.x, o.y);
                b.y = pack_bf16x2(o.z, o.w);
                *reinterpret_cast<uint2*>(dx16 + row * dm + i) = b;
            }
            p = make_float4(p.x + g.x * n.x, p.y + g.y * n.y, p.z + g.z * n.z, p.w + g.w * n.w);
        }
        *reinterpret_cast<float4*>(partial + (int64_t)blockIdx.x * dm + i) = p;
    }
}

// grad[j] += sum over blocks of partial[b][j], in block order
// out[c] += sum over b of partial[b][c], in a fixed order: a workgroup takes 64 columns; thread group g (of
// 4) sums rows g, g+4, g+8, ... in increasing order, then the four sums are added g = 0..3. Deterministic,
// and 4 x 64 lanes keep many rows in flight instead of one serial chain per column.
// Two such sums in one launch when out1 is given: blockIdx.y = 1 takes the partial rows that follow the first
// nblk and writes out1.
__global__ __launch_bounds__(256) void colsum_kernel(const float* partial, int nblk, int ncols, float* out0,
                                                     float* out1, int accumulate) {
    __shared__ float part[4][64];
    float* out = blockIdx.y ? out1 : out0;
    partial += (int64_t)blockIdx.y * nblk * ncols;
    const int cl = threadIdx.x & 63, g = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + cl;
    float s = 0.0f;
    if (c < ncols) {
#pragma unroll 8
        for (int b = g; b < nblk; b += 4) s += partial[(int64_t)b * ncols + c];
    }
    part[g][cl] = s;
    __syncthreads();
    if (g == 0 && c < ncols)  // (0 + sum when not accumulating: the value a zeroed out[c] would get)
        out[c] = (accumulate ? out[c] : 0.0f) + (((part[0][cl] + part[1][cl]) + part[2][cl]) + part[3][cl]);
}

// from d_act and the saved [gate | up] rows: d_gu = [d_gate | d_up] (gu and d_gu fp32, or both bf16)
template <bool kBF16>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const float* d_act, const void* gu, void* d_gu, int64_t rows,
                                                         int hid) {
    const int64_t n = rows * hid;
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < n; q += (int64_t)gridDim.x * 256) {
        const int64_t r = q / hid;
        const int i = (int)(q - r * hid);
        const float da = d_act[q];
        const float gate = load1(gu, r * 2 * hid + i, kBF16), up = load1(gu, r * 2 * hid + hid + i, kBF16);
        const float sig = 1.0f / (1.0f + expf(-gate));
        const float silu = gate * sig;
        const float d_up = da * silu;
        const float d_gate = da * up * sig * (1.0f + gate * (1.0f - sig));
        if constexpr (kBF16) {
            uint16_t* o = static_cast<uint16_t*>(d_gu);
            const bf16x2 v = __builtin_convertvector((floatx2){d_gate, d_up}, bf16x2);
            o[r * 2 * hid + i] = __builtin_bit_cast(uint32_t, v) & 0xffffu;
            o[r * 2 * hid + hid + i] = __builtin_bit_cast(uint32_t, v) >> 16;
        } else {
            float* o = static_cast<float*>(d_gu);
            o[r * 2 * hid + i] = d_gate;
            o[r * 2 * hid + hid + i] = d_up;
        }
    }
}

// bf16 [gate | up] and fp32 d_act -> bf16 d_gu, eight elements per thread and step (16-byte accesses,
// hid % 8 == 0); the same arithmetic as swiglu_bwd_kernel<true>
__global__ __launch_bounds__(256) void swiglu_bwd_bf16x8_kernel(const float* d_act, const uint16_t* gu, uint16_t* d_gu,
                                                                int64_t rows, int hid) {
    const int64_t n8 = rows * (hid / 8);
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < n8; q += (int64_t)gridDim.x * 256) {
        const int64_t r = q / (hid / 8);
        const int i = (int)(q - r * (hid / 8)) * 8;
        const float4 a0 = *reinterpret_cast<const float4*>(d_act + r * hid + i);
        const float4 a1 = *reinterpret_cast<const float4*>(d_act + r * hid + i + 4);
        const uint4 g = *reinterpret_cast<const uint4*>(gu + r * 2 * hid + i);
        const uint4 u = *reinterpret_cast<const uint4*>(gu + r * 2 * hid + hid + i);
        const float da[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
        uint32_t dg[4], du[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float d_gate[2], d_up[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float gate = __builtin_bit_cast(float, h ? (gw[e] & 0xffff0000u) : (gw[e] << 16));
                const float up = __builtin_bit_cast(float, h ? (uw[e] & 0xffff0000u) : (uw[e] << 16));
                const float sig = 1.0f / (1.0f + expf(-gate));
                const float silu = gate * sig;
                d_up[h] = da[2 * e + h] * silu;
                d_gate[h] = da[2 * e + h] * up * sig * (1.0f + gate * (1.0f - sig));
            }
            dg[e] = pack_bf16x2(d_gate[0], d_gate[1]);
            du[e] = pack_bf16x2(d_up[0], d_up[1]);
        }
        *reinterpret_cast<uint4*>(d_gu + r * 2 * hid + i) = make_uint4(dg[0], dg[1], dg[2], dg[3]);
        *reinterpret_cast<uint4*>(d_gu + r * 2 * hid + hid + i) = make_uint4(du[0], du[1], du[2], du[3]);
    }
}

// one workgroup per distinct token: E_grad[tok] += sum of dx rows pos[start[u]] .. pos[start[u+1]-1], in order
__global__ __launch_bounds__(256) void embed_bwd_kernel(const float* dx, const int32_t* uniq, const int32_t* start,
                                                        const int32_t* pos, float* g_embed, int dm) {
    const int u = blockIdx.x;
    const int64_t tok = uniq[u];
    for (int i = 4 * threadIdx.x; i < dm; i += 1024) {
        float4 acc = *reinterpret_cast<const float4*>(g_embed + tok * dm + i);
        for (int k = start[u]; k < start[u + 1]; ++k) {
            const float4 v = *reinterpret_cast<const float4*>(dx + (int64_t)pos[k] * dm + i);
            acc = make_float4(acc.x + v.x, acc.y + v.y, acc.z + v.z, acc.w + v.w);
        }
        *reinterpret_cast<float4*>(g_embed + tok * dm + i) = acc;
    }
}

// out = a + b (the block's residual gradient, OlmoBlock.cpp:32)
__global__ __launch_bounds__(256) void add_kernel(const float* a, const float* b, float* out, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        const float4 x = reinterpret_cast<const float4*>(a)[i], y = reinterpret_cast<const float4*>(b)[i];
        reinterpret_cast<float4*>(out)[i] = make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
    }
}

unsigned grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    return (unsigned)(b < 1 ? 1 : (b > 16384 ? 16384 : b));
}

}  // namespace

int launch_add(const float* a, const float* b, float* out, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(n / 4)), dim3(256), 0, s, a, b, out, n / 4);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

int launch_embed_gather(const int32_t* tok, const float* E, float* x, int rows, int dm, hipStream_t s) {
    hipLaunchKernelGGL(embed_gather_kernel, dim3(rows), dim3(256), 0, s, tok, E, x, dm);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

int launch_rmsnorm_rows(const float* a, const float* w, const float* res, float* out, uint16_t* out16, float* y_save,
                        float* rms_save, int rows, int dm, float eps, hipStream_t s) {
    if (dm == 2048)
        hipLaunchKernelGGL(rmsnorm_rows_reg_kernel<2>, dim3(rows), dim3(256), 0, s, a, w, res, out, out16, y_save,
                           rms_save, dm, eps);
    else
        hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(256), 0, s, a, w, res, out, out16, y_save, rms_save,
                           dm, eps);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

int launch_swiglu(const void* gu, void* act, int rows, int hid, int bf16, hipStream_t s) {
    const unsigned g = grid_for((int64_t)rows * hid / 4);
    if (bf16 && hid % 8 == 0)
        hipLaunchKernelGGL(swiglu_bf16x8_kernel, dim3(grid_for((int64_t)rows * hid / 8)), dim3(256), 0, s,
                           static_cast<const uint16_t*>(gu), static_cast<uint16_t*>(act), (int64_t)rows, hid);
    else if (bf16) hipLaunchKernelGGL(swiglu_kernel<true>, dim3(g), dim3(256), 0, s, gu, act, (int64_t)rows, hid);
    else hipLaunchKernelGGL(swiglu_kernel<false>, dim3(g), dim3(256), 0, s, gu, act, (int64_t)rows, hid);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

int launch_ce_loss(const float* logits, const int32_t* target, float* term, float* grad, float* loss, int rows, int V,
                   int count, hipStream_t s) {
    const float inv = count > 0 ? 1.0f / (float)count : __builtin_nanf("");  // 0 / 0 as in the reference
    const bool vec = V % 4 == 0 && ((uintptr_t)logits | (uintptr_t)grad) % 16 == 0;
    if (vec && V / 4 <= 1024 * kCeChunks)
        hipLaunchKernelGGL(ce_rows_reg_kernel<kCeChunks>, dim3(rows), dim3(1024), 0, s, logits, target, term, grad, V,
                           inv);
    else if (vec) hipLaunchKernelGGL(ce_rows_kernel<true>, dim3(rows), dim3(256), 0, s, logits, target, term, grad, V, inv);
    else hipLaunchKernelGGL(ce_rows_kernel<false>, dim3(rows), dim3(256), 0, s, logits, target, term, grad, V, inv);
    DT_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(ce_reduce_kernel, dim3(1), dim3(256), 0, s, term, (int64_t)rows, inv, loss);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

int rmsnorm_bwd_blocks(int rows) { return (rows + kRowsPerBlock - 1) / kRowsPerBlock; }

int launch_rmsnorm_bwd(const float* dy, const float* y, const float* rms, const float* w, const float* dx_add,
                       float* dx, float* partial, float* grad_w, int rows, int dm, hipStream_t s, bool accumulate,
                       uint16_t* dx16) {
    const int nblk = rmsnorm_bwd_blocks(rows);
    hipLaunchKernelGGL(rmsnorm_bwd_rows_kernel, dim3(nblk), dim3(256), 0, s, dy, y, rms, w, dx_add, dx, dx16, partial,
                       (int64_t)rows, dm);
    DT_HIP_TRY(hipGetLastError());
    if (!grad_w) return DT_OK;  // the caller sums the partial rows itself
    return launch_colsum(partial, nblk, dm, grad_w, s, accumulate);
}

int launch_colsum(const float* partial, int nblk, int ncols, float* out, hipStream_t s, bool accumulate,
                  float* out1) {
    hipLaunchKernelGGL(colsum_kernel, dim3((ncols + 63) / 64, out1 ? 2 : 1), dim3(256), 0, s, partial, nblk, ncols, out,
                       out1, accumulate ? 1 : 0);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

int launch_swiglu_bwd(const float* d_act, const void* gu, void* d_gu, int rows, int hid, int bf16, hipStream_t s) {
    const unsigned g = grid_for((int64_t)rows * hid);
    if (bf16 && hid % 8 == 0)
        hipLaunchKernelGGL(swiglu_bwd_bf16x8_kernel, dim3(grid_for((int64_t)rows * hid / 8)), dim3(256), 0, s, d_act,
                           static_cast<const uint16_t*>(gu), static_cast<uint16_t*>(d_gu), (int64_t)rows, hid);
    else if (bf16) hipLaunchKernelGGL(swiglu_bwd_kernel<true>, dim3(g), dim3(256), 0, s, d_act, gu, d_gu, (int64_t)rows, hid);
    else hipLaunchKernelGGL(swiglu_bwd_kernel<false>, dim3(g), dim3(256), 0, s, d_act, gu, d_gu, (int64_t)rows, hid);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

namespace {
// SGD on the listed rows of an embedding table, w -= lr * g (separate product and difference, as sgd4_kernel);
// with zero_rows set, the rows' gradients are cleared instead
__global__ __launch_bounds__(256) void embed_rows_kernel(float* w, float* g, const int32_t* rows, int dm, float lr,
                                                         int zero_rows) {
#pragma clang fp contract(off)
    const int64_t base = (int64_t)rows[blockIdx.x] * dm;
    float4* g4 = reinterpret_cast<float4*>(g + base);
    float4* w4 = reinterpret_cast<float4*>(w + base);
    for (int i = threadIdx.x; i < dm / 4; i += 256) {
        if (zero_rows) {
            g4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
            const float4 gv = g4[i];
            float4 wv = w4[i];
            wv.x = wv.x - lr * gv.x;
            wv.y = wv.y - lr * gv.y;
            wv.z = wv.z - lr * gv.z;
            wv.w = wv.w - lr * gv.w;
            w4[i] = wv;
        }
    }
}
}  // namespace

int launch_embed_rows(float* w, float* g, const int32_t* rows, int n_rows, int dm, float lr, bool zero_rows,
                      hipStream_t s) {
    if (n_rows == 0) return DT_OK;
    if (dm % 4 != 0 || (reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(g)) % 16 != 0)
        return set_error(DT_ERR_INVALID_ARG, "embedding rows: d_model %% 4 and 16-byte alignment required");
    hipLaunchKernelGGL(embed_rows_kernel, dim3(n_rows), dim3(256), 0, s, w, g, rows, dm, lr, zero_rows ? 1 : 0);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

int launch_embed_bwd(const float* dx, const int32_t* uniq, const int32_t* start, const int32_t* pos, int n_uniq,
                     float* g_embed, int dm, hipStream_t s) {
    if (n_uniq == 0) return DT_OK;
    hipLaunchKernelGGL(embed_bwd_kernel, dim3(n_uniq), dim3(256), 0, s, dx, uniq, start, pos, g_embed, dm);
    DT_HIP_TRY(hipGetLastError());
    return DT_OK;
}

}  // namespace dt
