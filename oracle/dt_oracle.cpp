// CPU oracle for the causal-attention path — TEST INFRASTRUCTURE ONLY.
//
// This file restates, on the CPU, the reference algorithms that the HIP kernels
// replace. It is linked only by the test suite, by __graft_entry__.smoke() and
// by bench.py's cpu_baseline leg, always to verify results (or as the timed CPU
// baseline), never as part of the product path.
//
// Functions and the reference code each one follows:
//   oracle_rope_tables            OlmoAttention.cpp:16-36    (fp64 angles, cast to fp32)
//   oracle_apply_rope             OlmoAttention.cpp:111-146  (rotate-half, position = t)
//   oracle_rmsnorm_forward        RMSNorm.cpp:15-22, RMSNorm.h:10 (x / sqrt(mean(x^2)+eps) * w)
//   oracle_flash_attention_forward FlashAttention.cpp:24-182 (256x256 tiles, tile-local max,
//                                  alpha/beta online rescale, l==0 -> zero row)
//   oracle_attention_layer_forward OlmoAttention.cpp:56-108  (projections, q/k norm over all
//                                  2048 features, RoPE, flash, o_proj)
//   oracle_sgemm_nt / _nn         stand-ins for the cblas_sgemm calls at FlashAttention.cpp:83,123
//                                  and xt::linalg::dot at OlmoAttention.cpp:68,74,80,104
//   oracle_flash_attention_backward FlashAttention.cpp:185-359 (D = O.dO, P from the saved m and l,
//                                  dS = P (dP - D) scale, 256x256 blocks)
//   oracle_apply_rope_backward    OlmoAttention.cpp:149-190  (transpose of the rotation)
//   oracle_rmsnorm_backward       RMSNorm.cpp:24-36          (c = mean(dy*y), n = y/w recomputed)
//   oracle_attention_layer_backward OlmoAttention.cpp:193-312 (o_proj, flash, RoPE, norms and
//                                  q/k/v projection backward; weight gradients accumulated)
//   oracle_mlp_forward            OlmoMlp.cpp:26-63          (SwiGLU: silu(x Wgate^T) * x Wup^T, Wdown)
//   oracle_model_forward          OlmoModel.cpp:25-48, OlmoBlock.cpp:13-21 (embedding, post-norm
//                                  blocks, final norm, LM head OlmoLmHead.cpp:11-28)
//   oracle_ce_loss                CrossEntropyLoss.cpp:8-43 and main.cpp:62-80 (loss with
//                                  ignore_index, and the softmax - onehot gradient / count)
//   oracle_model_backward         OlmoModel.cpp:50-67, OlmoBlock.cpp:23-30, OlmoMlp.cpp (backward),
//                                  OlmoLmHead.cpp:30-62 (all parameter gradients)
//
// Parity pins (checked in tests/test_oracle_pins.py): an fp64 full-softmax attention
// written independently in numpy, torch's scaled_dot_product_attention in fp64,
// HF transformers' Olmo2 rotate_half / apply_rotary_pos_emb and Olmo2Attention,
// torch.nn.functional.rms_norm in fp64, closed-form invariants (row 0, Q == 0,
// causality, RoPE identity at t=0, relative-position property, scale invariance)
// and brute force at T <= 8. oracle_set_mutation() plants known mistakes so that
// the tests can show each pin catches them.
//
// The BLAS summation order of the reference (whichever CBLAS it links) is not
// reproduced; parity with it is by tolerance.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

namespace {

int g_mutation = 0;  // 0 = faithful restatement; >0 = planted mistake (tests only)

constexpr float kNegInf = -std::numeric_limits<float>::infinity();

template <class F>
void parallel_for(int64_t n, int nthreads, F&& fn) {
    if (nthreads <= 1 || n <= 1) {
        for (int64_t i = 0; i < n; ++i) fn(i);
        return;
    }
    nthreads = (int)std::min<int64_t>(nthreads, n);
    std::vector<std::thread> pool;
    pool.reserve(nthreads);
    for (int t = 0; t < nthreads; ++t) {
        pool.emplace_back([&, t] {
            // contiguous blocks, like tbb::blocked_range over [0, n)
            int64_t lo = n * t / nthreads, hi = n * (t + 1) / nthreads;
            for (int64_t i = lo; i < hi; ++i) fn(i);
        });
    }
    for (auto& th : pool) th.join();
}

// C[i][j] = alpha * sum_k A[i][k] * B[j][k]    (row-major, "NoTrans, Trans")
void gemm_nt_serial(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                    float* C, int ldc) {
    int i = 0;
    for (; i + 4 <= M; i += 4) {
        const float* a0 = A + (int64_t)i * lda;
        const float* a1 = a0 + lda;
        const float* a2 = a1 + lda;
        const float* a3 = a2 + lda;
        int j = 0;
        for (; j + 2 <= N; j += 2) {
            const float* b0 = B + (int64_t)j * ldb;
            const float* b1 = b0 + ldb;
            float s00 = 0, s01 = 0, s10 = 0, s11 = 0, s20 = 0, s21 = 0, s30 = 0, s31 = 0;
            for (int k = 0; k < K; ++k) {
                float x0 = b0[k], x1 = b1[k];
                s00 += a0[k] * x0; s01 += a0[k] * x1;
                s10 += a1[k] * x0; s11 += a1[k] * x1;
                s20 += a2[k] * x0; s21 += a2[k] * x1;
                s30 += a3[k] * x0; s31 += a3[k] * x1;
            }
            float* c = C + (int64_t)i * ldc + j;
            c[0] = alpha * s00; c[1] = alpha * s01; c += ldc;
            c[0] = alpha * s10; c[1] = alpha * s11; c += ldc;
            c[0] = alpha * s20; c[1] = alpha * s21; c += ldc;
            c[0] = alpha * s30; c[1] = alpha * s31;
        }
        for (; j < N; ++j) {
            const float* b0 = B + (int64_t)j * ldb;
            float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            for (int k = 0; k < K; ++k) {
                s0 += a0[k] * b0[k]; s1 += a1[k] * b0[k]; s2 += a2[k] * b0[k]; s3 += a3[k] * b0[k];
            }
            C[(int64_t)i * ldc + j] = alpha * s0;
            C[(int64_t)(i + 1) * ldc + j] = alpha * s1;
            C[(int64_t)(i + 2) * ldc + j] = alpha * s2;
            C[(int64_t)(i + 3) * ldc + j] = alpha * s3;
        }
    }
    for (; i < M; ++i) {
        const float* a0 = A + (int64_t)i * lda;
        for (int j = 0; j < N; ++j) {
            const float* b0 = B + (int64_t)j * ldb;
            float s = 0;
            for (int k = 0; k < K; ++k) s += a0[k] * b0[k];
            C[(int64_t)i * ldc + j] = alpha * s;
        }
    }
}

// C[i][n] = beta * C[i][n] + sum_k A[k][i] * B[k][n]    (row-major, "Trans, NoTrans")
void gemm_tn_serial(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float beta, float* C,
                    int ldc) {
    for (int i = 0; i < M; ++i) {
        float* c = C + (int64_t)i * ldc;
        if (beta == 0.0f) std::fill(c, c + N, 0.0f);
        for (int k = 0; k < K; ++k) {
            const float av = A[(int64_t)k * lda + i];
            if (av == 0.0f) continue;
            const float* b = B + (int64_t)k * ldb;
            for (int n = 0; n < N; ++n) c[n] += av * b[n];
        }
    }
}

// C[i][n] = sum_k A[i][k] * B[k][n]    (row-major, "NoTrans, NoTrans"), beta = 0
void gemm_nn_serial(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C, int ldc) {
    for (int i = 0; i < M; ++i) {
        float* c = C + (int64_t)i * ldc;
        std::fill(c, c + N, 0.0f);
        const float* a = A + (int64_t)i * lda;
        for (int k = 0; k < K; ++k) {
            const float av = a[k];
            if (av == 0.0f) continue;
            const float* b = B + (int64_t)k * ldb;
            for (int n = 0; n < N; ++n) c[n] += av * b[n];
        }
    }
}

}  // namespace

extern "C" {

int oracle_version(void) { return 1; }

// Planted mistakes, for tests that show the pins catch them:
//   1 flash: drop beta in the online rescale     (FlashAttention.cpp:141-151)
//   2 flash: mask the diagonal (q_pos <= k_pos)   (FlashAttention.cpp:102)
//   3 rope:  flip the sign of the sin term         (OlmoAttention.cpp:131-140)
//   4 rope:  pair d with d+1 instead of d+64       (OlmoAttention.cpp:125)
//   5 norm:  normalise per head (128) instead of over all features (OlmoAttention.cpp:70)
//   6 norm:  drop eps                              (RMSNorm.cpp:18)
//   7 flash: drop the softmax scale                (FlashAttention.cpp:86)
//   8 flash backward: drop D = O . dO               (FlashAttention.cpp:232-238, 288-295)
//   9 rope backward: rotate forwards, not back      (OlmoAttention.cpp:174-182)
//  10 norm backward: drop the c = mean(dy * y) term (RMSNorm.cpp:26, 35)
//  11 flash backward: P without the 1 / l           (FlashAttention.cpp:272)
//  12 mlp: drop the sigmoid from SiLU               (OlmoMlp.cpp:47-52)
//  13 model: pre-norm blocks instead of post-norm   (OlmoBlock.cpp:13-21)
//  14 ce: count the ignore_index targets           (CrossEntropyLoss.cpp:28-30)
void oracle_set_mutation(int m) { g_mutation = m; }
int oracle_get_mutation(void) { return g_mutation; }

// RoPE tables, OlmoAttention.cpp:16-31: inv_freq[i] = 1 / theta^(2i/D) in fp64,
// angle[p][j] = p * inv_freq[j mod D/2] (halves duplicated by concatenate),
// sin/cos evaluated in fp64 and cast to fp32. Tables are [max_seq][D].
void oracle_rope_tables(float* sin_out, float* cos_out, int max_seq, int D, float theta) {
    const int half = D / 2;
    std::vector<double> inv_freq(half);
    for (int i = 0; i < half; ++i) {
        const double e = (double)(2 * i) / (double)D;  // arange(0, D, 2) / D
        inv_freq[i] = 1.0 / std::pow((double)theta, e);
    }
    for (int p = 0; p < max_seq; ++p) {
        for (int j = 0; j < D; ++j) {
            const double ang = (double)p * inv_freq[j % half];
            sin_out[(int64_t)p * D + j] = (float)std::sin(ang);
            cos_out[(int64_t)p * D + j] = (float)std::cos(ang);
        }
    }
}

// apply_rope, OlmoAttention.cpp:111-146. in/out are [B,T,H,D]; tables [>=T][D].
void oracle_apply_rope(const float* in, float* out, int B, int T, int H, int D, const float* sin_t,
                       const float* cos_t) {
    const int half = D / 2;
    const int pair = (g_mutation == 4) ? 1 : half;
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t)
            for (int h = 0; h < H; ++h) {
                const float* x = in + (((int64_t)b * T + t) * H + h) * D;
                float* y = out + (((int64_t)b * T + t) * H + h) * D;
                const float* c = cos_t + (int64_t)t * D;
                const float* s = sin_t + (int64_t)t * D;
                if (pair == half) {
                    for (int d = 0; d < half; ++d) {
                        const float sgn = (g_mutation == 3) ? -1.0f : 1.0f;
                        y[d] = x[d] * c[d] - sgn * x[d + half] * s[d];
                        y[d + half] = x[d + half] * c[d + half] + sgn * x[d] * s[d + half];
                    }
                } else {  // planted mistake 4: adjacent pairs
                    for (int d = 0; d < D; d += 2) {
                        y[d] = x[d] * c[d / 2] - x[d + 1] * s[d / 2];
                        y[d + 1] = x[d + 1] * c[d / 2] + x[d] * s[d / 2];
                    }
                }
            }
}

// RMSNorm::forward, RMSNorm.cpp:15-22 (eps RMSNorm.h:10): rms = sqrt(sum(x^2)/C + eps); y = (x / rms) * w.
// x, y are [rows][C]; rms_out (nullable) is [rows].
void oracle_rmsnorm_forward(const float* x, const float* w, float* y, float* rms_out, int rows, int C,
                            float eps) {
    if (g_mutation == 6) eps = 0.0f;
    const int group = (g_mutation == 5) ? 128 : C;
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (int64_t)r * C;
        float* yr = y + (int64_t)r * C;
        for (int g0 = 0; g0 < C; g0 += group) {
            float ss = 0.0f;
            for (int c = g0; c < g0 + group; ++c) ss += xr[c] * xr[c];
            const float rms = std::sqrt(ss / (float)group + eps);
            if (rms_out && g0 == 0) rms_out[r] = rms;
            for (int c = g0; c < g0 + group; ++c) yr[c] = (xr[c] / rms) * w[c];
        }
    }
}

// flash_attention_forward, FlashAttention.cpp:24-182. Q, K, V, O are [B,T,H,D] row-major;
// m, l are [B,T,H]. Threads split the B*H (batch, head) items like the reference's
// tbb::parallel_for over bh (FlashAttention.cpp:43-45).
void oracle_flash_attention_forward(const float* Q, const float* K, const float* V, float* O, float* m_out,
                                    float* l_out, int B, int T, int H, int D, float scale, int causal,
                                    int nthreads) {
    constexpr int BQ = 256, BKV = 256;  // FlashAttention.cpp:21-22
    const int ld = H * D;
    auto at = [&](const float* base, int b, int t, int h) { return base + ((int64_t)b * T + t) * ld + (int64_t)h * D; };
    parallel_for((int64_t)B * H, nthreads, [&](int64_t bh) {
        const int b = (int)(bh / H), h = (int)(bh % H);
        std::vector<float> S((size_t)BQ * BKV), P((size_t)BQ * BKV), PV((size_t)BQ * D);
        std::vector<float> m(BQ), l(BQ), Ob((size_t)BQ * D), m_loc(BQ), l_loc(BQ);
        for (int q0 = 0; q0 < T; q0 += BQ) {
            const int Br = std::min(BQ, T - q0);
            std::fill(m.begin(), m.begin() + Br, kNegInf);
            std::fill(l.begin(), l.begin() + Br, 0.0f);
            std::fill(Ob.begin(), Ob.begin() + (size_t)Br * D, 0.0f);
            for (int k0 = 0; k0 < T; k0 += BKV) {
                const int Bc = std::min(BKV, T - k0);
                if (causal && q0 < k0) continue;  // whole tile above the diagonal
                // S = scale * Q_blk K_blk^T (sgemm alpha), FlashAttention.cpp:83-91
                const float alpha_s = (g_mutation == 7) ? 1.0f : scale;
                gemm_nt_serial(Br, Bc, D, alpha_s, at(Q, b, q0, h), ld, at(K, b, k0, h), ld, S.data(), BKV);
                // mask, tile-local max, P = exp(S - m_local), l_local; FlashAttention.cpp:94-120
                for (int i = 0; i < Br; ++i) {
                    float* s = S.data() + (size_t)i * BKV;
                    float* p = P.data() + (size_t)i * BKV;
                    m_loc[i] = kNegInf;
                    for (int j = 0; j < Bc; ++j) {
                        const int qp = q0 + i, kp = k0 + j;
                        const bool masked = causal && ((g_mutation == 2) ? (qp <= kp) : (qp < kp));
                        if (masked) s[j] = kNegInf;
                        else m_loc[i] = std::max(m_loc[i], s[j]);
                    }
                    l_loc[i] = 0.0f;
                    for (int j = 0; j < Bc; ++j) {
                        if (s[j] > kNegInf) {
                            const float e = std::exp(s[j] - m_loc[i]);
                            p[j] = e;
                            l_loc[i] += e;
                        } else {
                            p[j] = 0.0f;
                        }
                    }
                }
                // PV = P V_blk, FlashAttention.cpp:123-131
                gemm_nn_serial(Br, D, Bc, P.data(), BKV, at(V, b, k0, h), ld, PV.data(), D);
                // online rescale, FlashAttention.cpp:134-156
                for (int i = 0; i < Br; ++i) {
                    const float m_new = std::max(m[i], m_loc[i]);
                    const float a = (m[i] > kNegInf) ? std::exp(m[i] - m_new) : 0.0f;
                    float be = (m_loc[i] > kNegInf) ? std::exp(m_loc[i] - m_new) : 0.0f;
                    if (g_mutation == 1) be = 1.0f;
                    l[i] = l[i] * a + l_loc[i] * be;
                    float* o = Ob.data() + (size_t)i * D;
                    const float* pv = PV.data() + (size_t)i * D;
                    for (int d = 0; d < D; ++d) o[d] = o[d] * a + pv[d] * be;
                    m[i] = m_new;
                }
            }
            // finalize, FlashAttention.cpp:159-175
            for (int i = 0; i < Br; ++i) {
                const int64_t idx = ((int64_t)b * T + q0 + i) * H + h;
                m_out[idx] = m[i];
                l_out[idx] = l[i];
                float* dst = O + idx * D;
                if (l[i] > 0.0f) {
                    for (int d = 0; d < D; ++d) dst[d] = Ob[(size_t)i * D + d] / l[i];
                } else {
                    for (int d = 0; d < D; ++d) dst[d] = 0.0f;
                }
            }
        }
    });
}

// C = alpha * A B^T, row-major, threaded over row blocks of C.
void oracle_sgemm_nt(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb, float* C,
                     int ldc, int nthreads) {
    const int rb = 32;
    const int nblk = (M + rb - 1) / rb;
    parallel_for(nblk, nthreads, [&](int64_t blk) {
        const int i0 = (int)blk * rb, rows = std::min(rb, M - i0);
        // block over N to keep a panel of B in cache
        for (int j0 = 0; j0 < N; j0 += 256) {
            const int cols = std::min(256, N - j0);
            gemm_nt_serial(rows, cols, K, alpha, A + (int64_t)i0 * lda, lda, B + (int64_t)j0 * ldb, ldb,
                           C + (int64_t)i0 * ldc + j0, ldc);
        }
    });
}

// OlmoAttention::forward, OlmoAttention.cpp:56-108, for d_model = H*D with D = 128.
// x, out are [B,T,d_model]; weights are [d_model][d_model] stored [out][in] (y = x W^T);
// q_norm_w, k_norm_w are [d_model]. rope tables [>=T][D]. Optional saved state:
// q_rope, k_rope, v_out, attn_out [B,T,H,D], m, l [B,T,H] (each nullable).
void oracle_attention_layer_forward(const float* x, const float* wq, const float* wk, const float* wv,
                                    const float* wo, const float* q_norm_w, const float* k_norm_w,
                                    const float* sin_t, const float* cos_t, float* out, int B, int T, int H,
                                    int D, float eps, int nthreads, float* q_rope, float* k_rope, float* v_out,
                                    float* attn_out, float* m_out, float* l_out) {
    const int dm = H * D;
    const int64_t rows = (int64_t)B * T;
    const size_t n = (size_t)rows * dm;
    std::vector<float> q(n), k(n), v(n), qn(n), kn(n), qr(n), kr(n), o(n);
    std::vector<float> mm((size_t)rows * H), ll((size_t)rows * H);
    oracle_sgemm_nt((int)rows, dm, dm, 1.0f, x, dm, wq, dm, q.data(), dm, nthreads);   // :68
    oracle_rmsnorm_forward(q.data(), q_norm_w, qn.data(), nullptr, (int)rows, dm, eps); // :70
    oracle_sgemm_nt((int)rows, dm, dm, 1.0f, x, dm, wk, dm, k.data(), dm, nthreads);   // :74
    oracle_rmsnorm_forward(k.data(), k_norm_w, kn.data(), nullptr, (int)rows, dm, eps); // :76
    oracle_sgemm_nt((int)rows, dm, dm, 1.0f, x, dm, wv, dm, v.data(), dm, nthreads);   // :80
    oracle_apply_rope(qn.data(), qr.data(), B, T, H, D, sin_t, cos_t);                  // :87
    oracle_apply_rope(kn.data(), kr.data(), B, T, H, D, sin_t, cos_t);                  // :88
    const float scale = 1.0f / std::sqrt((float)D);                                      // :91
    oracle_flash_attention_forward(qr.data(), kr.data(), v.data(), o.data(), mm.data(), ll.data(), B, T, H, D,
                                   scale, 1, nthreads);                                  // :94
    oracle_sgemm_nt((int)rows, dm, dm, 1.0f, o.data(), dm, wo, dm, out, dm, nthreads); // :104
    if (q_rope) std::memcpy(q_rope, qr.data(), n * sizeof(float));
    if (k_rope) std::memcpy(k_rope, kr.data(), n * sizeof(float));
    if (v_out) std::memcpy(v_out, v.data(), n * sizeof(float));
    if (attn_out) std::memcpy(attn_out, o.data(), n * sizeof(float));
    if (m_out) std::memcpy(m_out, mm.data(), mm.size() * sizeof(float));
    if (l_out) std::memcpy(l_out, ll.data(), ll.size() * sizeof(float));
}


// flash_attention_backward, FlashAttention.cpp:185-359. dO, O, Q, K, V, dQ, dK, dV are [B,T,H,D];
// m, l are the forward's [B,T,H] statistics. Per (batch, head) and 256-query block:
// D_i = O_i . dO_i (:232-238); per 256-key block (skipped when causal and q_start < k_start, :247):
// S = scale Q K^T (:249-258), P = exp(S - m) / l with masked entries 0 (:260-275),
// dP = dO V^T (:277-286), dS = P (dP - D) scale (:288-295), dV += P^T dO (:297-313),
// dQ += dS K (:316-325), dK += dS^T Q (:327-343).
void oracle_flash_attention_backward(const float* dO, const float* O, const float* m, const float* l,
                                     const float* Q, const float* K, const float* V, float* dQ, float* dK,
                                     float* dV, int B, int T, int H, int D, float scale, int causal,
                                     int nthreads) {
    constexpr int BQ = 256, BKV = 256;  // FlashAttention.cpp:21-22
    const int ld = H * D;
    auto at = [&](const float* base, int b, int t, int h) { return base + ((int64_t)b * T + t) * ld + (int64_t)h * D; };
    auto atw = [&](float* base, int b, int t, int h) { return base + ((int64_t)b * T + t) * ld + (int64_t)h * D; };
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t)
            for (int h = 0; h < H; ++h) {
                std::fill(atw(dQ, b, t, h), atw(dQ, b, t, h) + D, 0.0f);
                std::fill(atw(dK, b, t, h), atw(dK, b, t, h) + D, 0.0f);
                std::fill(atw(dV, b, t, h), atw(dV, b, t, h) + D, 0.0f);
            }
    parallel_for((int64_t)B * H, nthreads, [&](int64_t bh) {
        const int b = (int)(bh / H), h = (int)(bh % H);
        std::vector<float> S((size_t)BQ * BKV), P((size_t)BQ * BKV), dP((size_t)BQ * BKV), dS((size_t)BQ * BKV);
        std::vector<float> Di(BQ), dQb((size_t)BQ * D), dKb((size_t)BKV * D), dVb((size_t)BKV * D);
        for (int q0 = 0; q0 < T; q0 += BQ) {
            const int Br = std::min(BQ, T - q0);
            for (int i = 0; i < Br; ++i) {
                const float* o = at(O, b, q0 + i, h);
                const float* g = at(dO, b, q0 + i, h);
                float acc = 0.0f;
                for (int d = 0; d < D; ++d) acc += o[d] * g[d];
                Di[i] = (g_mutation == 8) ? 0.0f : acc;
            }
            std::fill(dQb.begin(), dQb.begin() + (size_t)Br * D, 0.0f);
            for (int k0 = 0; k0 < T; k0 += BKV) {
                const int Bc = std::min(BKV, T - k0);
                if (causal && q0 < k0) continue;
                gemm_nt_serial(Br, Bc, D, scale, at(Q, b, q0, h), ld, at(K, b, k0, h), ld, S.data(), BKV);
                for (int i = 0; i < Br; ++i) {
                    const int64_t si = ((int64_t)b * T + q0 + i) * H + h;
                    const float mi = m[si];
                    const float li = (g_mutation == 11) ? 1.0f : l[si];
                    for (int j = 0; j < Bc; ++j) {
                        const bool masked = causal && (q0 + i < k0 + j);
                        P[(size_t)i * BKV + j] = masked ? 0.0f : std::exp(S[(size_t)i * BKV + j] - mi) / li;
                    }
                }
                gemm_nt_serial(Br, Bc, D, 1.0f, at(dO, b, q0, h), ld, at(V, b, k0, h), ld, dP.data(), BKV);
                for (int i = 0; i < Br; ++i)
                    for (int j = 0; j < Bc; ++j)
                        dS[(size_t)i * BKV + j] = P[(size_t)i * BKV + j] * (dP[(size_t)i * BKV + j] - Di[i]) * scale;
                // dV_blk = P^T dO, accumulated into dV
                gemm_tn_serial(Bc, D, Br, P.data(), BKV, at(dO, b, q0, h), ld, 0.0f, dVb.data(), D);
                for (int j = 0; j < Bc; ++j) {
                    float* dst = atw(dV, b, k0 + j, h);
                    for (int d = 0; d < D; ++d) dst[d] += dVb[(size_t)j * D + d];
                }
                // dQ_blk += dS K
                for (int i = 0; i < Br; ++i) {
                    float* dq = dQb.data() + (size_t)i * D;
                    for (int j = 0; j < Bc; ++j) {
                        const float w = dS[(size_t)i * BKV + j];
                        if (w == 0.0f) continue;
                        const float* kr = at(K, b, k0 + j, h);
                        for (int d = 0; d < D; ++d) dq[d] += w * kr[d];
                    }
                }
                // dK_blk = dS^T Q, accumulated into dK
                gemm_tn_serial(Bc, D, Br, dS.data(), BKV, at(Q, b, q0, h), ld, 0.0f, dKb.data(), D);
                for (int j = 0; j < Bc; ++j) {
                    float* dst = atw(dK, b, k0 + j, h);
                    for (int d = 0; d < D; ++d) dst[d] += dKb[(size_t)j * D + d];
                }
            }
            for (int i = 0; i < Br; ++i) std::memcpy(atw(dQ, b, q0 + i, h), dQb.data() + (size_t)i * D, D * sizeof(float));
        }
    });
}

// apply_rope_backward, OlmoAttention.cpp:149-190: the transpose of the rotation,
// d_in[d] = d_out[d] cos[d] + d_out[d+64] sin[d+64], d_in[d+64] = -d_out[d] sin[d] + d_out[d+64] cos[d+64].
void oracle_apply_rope_backward(const float* d_out, float* d_in, int B, int T, int H, int D, const float* sin_t,
                                const float* cos_t) {
    const int half = D / 2;
    const float sgn = (g_mutation == 9) ? -1.0f : 1.0f;
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t)
            for (int h = 0; h < H; ++h) {
                const float* g = d_out + (((int64_t)b * T + t) * H + h) * D;
                float* y = d_in + (((int64_t)b * T + t) * H + h) * D;
                const float* c = cos_t + (int64_t)t * D;
                const float* s = sin_t + (int64_t)t * D;
                for (int d = 0; d < half; ++d) {
                    y[d] = g[d] * c[d] + sgn * g[d + half] * s[d + half];
                    y[d + half] = -sgn * g[d] * s[d] + g[d + half] * c[d + half];
                }
            }
}

// RMSNorm::backward, RMSNorm.cpp:24-36, from the forward's saved output y and rms:
// c = mean(dy * y) over the row; n = y / w (recomputed, :29); dw += sum over rows of dy * n;
// dx = (w * dy - n * c) / rms. x-shaped arrays are [rows][C]; dw is accumulated (+=).
void oracle_rmsnorm_backward(const float* dy, const float* y, const float* rms, const float* w, float* dx,
                             float* dw, int rows, int C) {
    for (int r = 0; r < rows; ++r) {
        const float* g = dy + (int64_t)r * C;
        const float* yr = y + (int64_t)r * C;
        float acc = 0.0f;
        for (int c = 0; c < C; ++c) acc += g[c] * yr[c];
        const float cm = (g_mutation == 10) ? 0.0f : acc / (float)C;
        float* out = dx + (int64_t)r * C;
        for (int c = 0; c < C; ++c) {
            const float n = yr[c] / w[c];
            dw[c] += g[c] * n;
            out[c] = (w[c] * g[c] - n * cm) / rms[r];
        }
    }
}

// C = A B (row-major, "NoTrans, NoTrans"), threaded over row blocks of C.
void oracle_sgemm_nn(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C, int ldc,
                     int nthreads) {
    const int rb = 16;
    parallel_for((M + rb - 1) / rb, nthreads, [&](int64_t blk) {
        const int i0 = (int)blk * rb, rows = std::min(rb, M - i0);
        gemm_nn_serial(rows, N, K, A + (int64_t)i0 * lda, lda, B, ldb, C + (int64_t)i0 * ldc, ldc);
    });
}

// C += A^T B (row-major, "Trans, NoTrans", beta = 1), threaded over row blocks of C.
void oracle_sgemm_tn_acc(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C, int ldc,
                         int nthreads) {
    const int rb = 16;
    parallel_for((M + rb - 1) / rb, nthreads, [&](int64_t blk) {
        const int i0 = (int)blk * rb, rows = std::min(rb, M - i0);
        gemm_tn_serial(rows, N, K, A + i0, lda, B, ldb, 1.0f, C + (int64_t)i0 * ldc, ldc);
    });
}

// OlmoAttention::backward, OlmoAttention.cpp:193-312, for d_model = H*D with D = 128. The
// forward's saved state (OlmoAttention.h:28-38) is recomputed from x and the weights. d_out and
// d_x are [B,T,d_model]; the weight gradients are accumulated (+=, the reference's beta = 1 at
// :207-211, :257-277, and RMSNorm.cpp:31): dwq/dwk/dwv/dwo [d_model][d_model], dq_norm/dk_norm [d_model].
void oracle_attention_layer_backward(const float* x, const float* wq, const float* wk, const float* wv,
                                     const float* wo, const float* q_norm_w, const float* k_norm_w,
                                     const float* sin_t, const float* cos_t, const float* d_out, float* d_x,
                                     float* dwq, float* dwk, float* dwv, float* dwo, float* dq_norm,
                                     float* dk_norm, int B, int T, int H, int D, float eps, int nthreads) {
    const int dm = H * D;
    const int rows = B * T;
    const size_t n = (size_t)rows * dm;
    // forward, keeping what the reference saves (OlmoAttention.cpp:64-100)
    std::vector<float> q(n), k(n), v(n), qn(n), kn(n), qr(n), kr(n), o(n), q_rms(rows), k_rms(rows);
    std::vector<float> mm((size_t)rows * H), ll((size_t)rows * H);
    oracle_sgemm_nt(rows, dm, dm, 1.0f, x, dm, wq, dm, q.data(), dm, nthreads);
    oracle_rmsnorm_forward(q.data(), q_norm_w, qn.data(), q_rms.data(), rows, dm, eps);
    oracle_sgemm_nt(rows, dm, dm, 1.0f, x, dm, wk, dm, k.data(), dm, nthreads);
    oracle_rmsnorm_forward(k.data(), k_norm_w, kn.data(), k_rms.data(), rows, dm, eps);
    oracle_sgemm_nt(rows, dm, dm, 1.0f, x, dm, wv, dm, v.data(), dm, nthreads);
    oracle_apply_rope(qn.data(), qr.data(), B, T, H, D, sin_t, cos_t);
    oracle_apply_rope(kn.data(), kr.data(), B, T, H, D, sin_t, cos_t);
    const float scale = 1.0f / std::sqrt((float)D);
    oracle_flash_attention_forward(qr.data(), kr.data(), v.data(), o.data(), mm.data(), ll.data(), B, T, H, D,
                                   scale, 1, nthreads);
    // step 1, :198-217: dWo += d_out^T attn; d_attn = d_out Wo
    oracle_sgemm_tn_acc(dm, dm, rows, d_out, dm, o.data(), dm, dwo, dm, nthreads);
    std::vector<float> d_attn(n), dqr(n), dkr(n), dv(n), dqn(n), dkn(n), dq(n), dk(n);
    oracle_sgemm_nn(rows, dm, dm, d_out, dm, wo, dm, d_attn.data(), dm, nthreads);
    // step 2, :219-232: flash backward from the saved statistics
    oracle_flash_attention_backward(d_attn.data(), o.data(), mm.data(), ll.data(), qr.data(), kr.data(), v.data(),
                                    dqr.data(), dkr.data(), dv.data(), B, T, H, D, scale, 1, nthreads);
    // step 3, :234-236: RoPE backward
    oracle_apply_rope_backward(dqr.data(), dqn.data(), B, T, H, D, sin_t, cos_t);
    oracle_apply_rope_backward(dkr.data(), dkn.data(), B, T, H, D, sin_t, cos_t);
    // step 4, :238-244: q/k RMSNorm backward
    oracle_rmsnorm_backward(dqn.data(), qn.data(), q_rms.data(), q_norm_w, dq.data(), dq_norm, rows, dm);
    oracle_rmsnorm_backward(dkn.data(), kn.data(), k_rms.data(), k_norm_w, dk.data(), dk_norm, rows, dm);
    // step 5, :246-277: dW += d_proj^T x
    oracle_sgemm_tn_acc(dm, dm, rows, dq.data(), dm, x, dm, dwq, dm, nthreads);
    oracle_sgemm_tn_acc(dm, dm, rows, dk.data(), dm, x, dm, dwk, dm, nthreads);
    oracle_sgemm_tn_acc(dm, dm, rows, dv.data(), dm, x, dm, dwv, dm, nthreads);
    // :279-309: d_x = dq Wq + dk Wk + dv Wv
    std::vector<float> t1(n);
    oracle_sgemm_nn(rows, dm, dm, dq.data(), dm, wq, dm, d_x, dm, nthreads);
    oracle_sgemm_nn(rows, dm, dm, dk.data(), dm, wk, dm, t1.data(), dm, nthreads);
    for (size_t i = 0; i < n; ++i) d_x[i] += t1[i];
    oracle_sgemm_nn(rows, dm, dm, dv.data(), dm, wv, dm, t1.data(), dm, nthreads);
    for (size_t i = 0; i < n; ++i) d_x[i] += t1[i];
}


// ------------------------------------------------------------------------------------------------ model
// Per-layer parameter order of the model functions below (file names of OlmoBlock / OlmoAttention /
// OlmoMlp, OlmoBlock.cpp:5-11, OlmoAttention.cpp:39-53, OlmoMlp.cpp:9-24):
//   0 self_attn.q_proj  1 self_attn.k_proj  2 self_attn.v_proj  3 self_attn.o_proj
//   4 self_attn.q_norm  5 self_attn.k_norm  6 post_attention_layernorm
//   7 mlp.gate_proj     8 mlp.up_proj       9 mlp.down_proj     10 post_feedforward_layernorm
constexpr int kLayerParams = 11;

// OlmoMlp::forward, OlmoMlp.cpp:26-63: up = x Wup^T, gate = x Wgate^T, act = gate / (1 + exp(-gate)) * up,
// out = act Wdown^T. x [rows][dm], Wup/Wgate [hid][dm], Wdown [dm][hid]. gate/up/act (nullable) keep state.
void oracle_mlp_forward(const float* x, const float* w_gate, const float* w_up, const float* w_down, float* out,
                        int rows, int dm, int hid, int nthreads, float* gate_out, float* up_out, float* act_out) {
    std::vector<float> up((size_t)rows * hid), gate((size_t)rows * hid), act((size_t)rows * hid);
    oracle_sgemm_nt(rows, hid, dm, 1.0f, x, dm, w_up, dm, up.data(), hid, nthreads);
    oracle_sgemm_nt(rows, hid, dm, 1.0f, x, dm, w_gate, dm, gate.data(), hid, nthreads);
    for (size_t i = 0; i < act.size(); ++i) {
        const float g = gate[i];
        const float silu = (g_mutation == 12) ? g : g / (1.0f + std::exp(-g));
        act[i] = silu * up[i];
    }
    oracle_sgemm_nt(rows, dm, hid, 1.0f, act.data(), hid, w_down, hid, out, dm, nthreads);
    if (gate_out) std::memcpy(gate_out, gate.data(), gate.size() * sizeof(float));
    if (up_out) std::memcpy(up_out, up.data(), up.size() * sizeof(float));
    if (act_out) std::memcpy(act_out, act.data(), act.size() * sizeof(float));
}

// OlmoModel::forward, OlmoModel.cpp:25-48: embedding rows, n_layers post-norm blocks
// (OlmoBlock.cpp:13-21: h = x + N_attn(attn(x)); y = h + N_mlp(mlp(h))), final norm, LM head.
// tokens [B][T]; embed [V][dm]; layers: n_layers * 11 pointers in the order above; lm_head [V][dm];
// logits [B][T][V]. hid is the MLP width (8192 in the reference).
void oracle_model_forward(const int32_t* tokens, const float* embed, const float* const* layers,
                          const float* final_norm, const float* lm_head, float* logits, int B, int T, int dm,
                          int hid, int V, int n_layers, float eps, int nthreads) {
    const int rows = B * T, H = dm / 128;
    const size_t n = (size_t)rows * dm;
    std::vector<float> x(n), a(n), na(n), h(n), m(n), nm(n);
    for (int r = 0; r < rows; ++r) std::memcpy(&x[(size_t)r * dm], embed + (int64_t)tokens[r] * dm, dm * sizeof(float));
    std::vector<float> sin_t((size_t)T * 128), cos_t((size_t)T * 128);
    oracle_rope_tables(sin_t.data(), cos_t.data(), T, 128, 500000.0f);
    for (int i = 0; i < n_layers; ++i) {
        const float* const* p = layers + (size_t)i * kLayerParams;
        if (g_mutation == 13) {  // planted mistake: pre-norm blocks
            oracle_rmsnorm_forward(x.data(), p[6], na.data(), nullptr, rows, dm, eps);
            oracle_attention_layer_forward(na.data(), p[0], p[1], p[2], p[3], p[4], p[5], sin_t.data(), cos_t.data(),
                                           a.data(), B, T, H, 128, eps, nthreads, nullptr, nullptr, nullptr, nullptr,
                                           nullptr, nullptr);
            for (size_t j = 0; j < n; ++j) h[j] = x[j] + a[j];
            oracle_rmsnorm_forward(h.data(), p[10], nm.data(), nullptr, rows, dm, eps);
            oracle_mlp_forward(nm.data(), p[7], p[8], p[9], m.data(), rows, dm, hid, nthreads, nullptr, nullptr, nullptr);
            for (size_t j = 0; j < n; ++j) x[j] = h[j] + m[j];
            continue;
        }
        oracle_attention_layer_forward(x.data(), p[0], p[1], p[2], p[3], p[4], p[5], sin_t.data(), cos_t.data(),
                                       a.data(), B, T, H, 128, eps, nthreads, nullptr, nullptr, nullptr, nullptr,
                                       nullptr, nullptr);
        oracle_rmsnorm_forward(a.data(), p[6], na.data(), nullptr, rows, dm, eps);
        for (size_t j = 0; j < n; ++j) h[j] = x[j] + na[j];
        oracle_mlp_forward(h.data(), p[7], p[8], p[9], m.data(), rows, dm, hid, nthreads, nullptr, nullptr, nullptr);
        oracle_rmsnorm_forward(m.data(), p[10], nm.data(), nullptr, rows, dm, eps);
        for (size_t j = 0; j < n; ++j) x[j] = h[j] + nm[j];
    }
    oracle_rmsnorm_forward(x.data(), final_norm, na.data(), nullptr, rows, dm, eps);
    oracle_sgemm_nt(rows, V, dm, 1.0f, na.data(), dm, lm_head, dm, logits, V, nthreads);
}

// ce_loss, CrossEntropyLoss.cpp:8-43, and the gradient main.cpp:62-80 builds from its probs:
// loss = mean over (b, s < T-1) with tokens[b][s+1] != ignore of log(sum_v exp(l - max)) - (l[target] - max);
// d_logits (nullable) = (softmax - onehot(target)) / count at (b, s) for those positions, 0 elsewhere
// (pad targets and the last position). Returns the loss; count is written to *count_out (nullable).
float oracle_ce_loss(const float* logits, const int32_t* tokens, int B, int T, int V, int ignore_index,
                     float* d_logits, int* count_out) {
    double total = 0.0;  // the reference accumulates in float; a double sum keeps the oracle order-robust
    int count = 0;
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < T; ++s) {
            const float* l = logits + ((int64_t)b * T + s) * V;
            float* g = d_logits ? d_logits + ((int64_t)b * T + s) * V : nullptr;
            const bool has_target = s + 1 < T && (g_mutation == 14 || tokens[b * T + s + 1] != ignore_index);
            if (!has_target) {
                if (g) std::fill(g, g + V, 0.0f);
                continue;
            }
            float mx = l[0];
            for (int v = 1; v < V; ++v) mx = std::max(mx, l[v]);
            float se = 0.0f;
            for (int v = 0; v < V; ++v) se += std::exp(l[v] - mx);
            const int tgt = tokens[b * T + s + 1];
            total += (double)std::log(se) - (double)(l[tgt] - mx);
            ++count;
            if (g) {
                for (int v = 0; v < V; ++v) g[v] = std::exp(l[v] - mx) / se;
                g[tgt] -= 1.0f;
            }
        }
    // with no target at all the reference divides 0 by 0 (CrossEntropyLoss.cpp:40; main.cpp:88 divides the
    // zeroed probs by a zero count): the loss and every gradient element are NaN
    const float nan = std::numeric_limits<float>::quiet_NaN();
    if (d_logits) {
        const float inv = count > 0 ? 1.0f / (float)count : nan;
        for (size_t i = 0; i < (size_t)B * T * V; ++i) d_logits[i] *= inv;
    }
    if (count_out) *count_out = count;
    return count > 0 ? (float)(total / count) : nan;
}


// OlmoModel::backward, OlmoModel.cpp:50-67, after a forward on tokens (recomputed here, keeping what the
// reference's layers save). d_logits [B][T][V]. grads: the same pointer layout as the parameters
// (embed, n_layers * 11 in the order above, final_norm, lm_head), accumulated (+=).
//   LM head (OlmoLmHead.cpp:30-62): dW += d^T y_final, d_y = d W
//   final norm, then per block in reverse (OlmoBlock.cpp:23-30): d_m = N_pf'(d), MLP backward
//   (OlmoMlp.cpp:65-160: dWdown += d_m^T act, d_act = d_m Wdown, d_up = d_act silu(gate),
//   d_gate = d_act up sig (1 + gate (1 - sig)), dWgate += d_gate^T h, dWup += d_up^T h,
//   d_h = d_gate Wgate + d_up Wup + d), d_a = N_pa'(d_h), d = attn'(d_a) + d_h
//   embedding (OlmoModel.cpp:57-66): grad[token] += d rows
void oracle_model_backward(const int32_t* tokens, const float* embed, const float* const* layers,
                           const float* final_norm, const float* lm_head, const float* d_logits, float* g_embed,
                           float* const* g_layers, float* g_final_norm, float* g_lm_head, int B, int T, int dm,
                           int hid, int V, int n_layers, float eps, int nthreads) {
    const int rows = B * T, H = dm / 128;
    const size_t n = (size_t)rows * dm, nh = (size_t)rows * hid;
    std::vector<float> sin_t((size_t)T * 128), cos_t((size_t)T * 128);
    oracle_rope_tables(sin_t.data(), cos_t.data(), T, 128, 500000.0f);
    // forward with saved state
    std::vector<std::vector<float>> xin(n_layers, std::vector<float>(n)), ypa(n_layers, std::vector<float>(n)),
        h(n_layers, std::vector<float>(n)), ypf(n_layers, std::vector<float>(n)), gate(n_layers, std::vector<float>(nh)),
        up(n_layers, std::vector<float>(nh)), act(n_layers, std::vector<float>(nh));
    std::vector<std::vector<float>> rpa(n_layers, std::vector<float>(rows)), rpf(n_layers, std::vector<float>(rows));
    std::vector<float> x(n), a(n), m(n), yf(n), rf(rows);
    for (int r = 0; r < rows; ++r) std::memcpy(&x[(size_t)r * dm], embed + (int64_t)tokens[r] * dm, dm * sizeof(float));
    for (int i = 0; i < n_layers; ++i) {
        const float* const* p = layers + (size_t)i * kLayerParams;
        xin[i] = x;
        oracle_attention_layer_forward(x.data(), p[0], p[1], p[2], p[3], p[4], p[5], sin_t.data(), cos_t.data(),
                                       a.data(), B, T, H, 128, eps, nthreads, nullptr, nullptr, nullptr, nullptr,
                                       nullptr, nullptr);
        oracle_rmsnorm_forward(a.data(), p[6], ypa[i].data(), rpa[i].data(), rows, dm, eps);
        for (size_t j = 0; j < n; ++j) h[i][j] = x[j] + ypa[i][j];
        oracle_mlp_forward(h[i].data(), p[7], p[8], p[9], m.data(), rows, dm, hid, nthreads, gate[i].data(),
                           up[i].data(), act[i].data());
        oracle_rmsnorm_forward(m.data(), p[10], ypf[i].data(), rpf[i].data(), rows, dm, eps);
        for (size_t j = 0; j < n; ++j) x[j] = h[i][j] + ypf[i][j];
    }
    oracle_rmsnorm_forward(x.data(), final_norm, yf.data(), rf.data(), rows, dm, eps);
    // LM head and final norm
    oracle_sgemm_tn_acc(V, dm, rows, d_logits, V, yf.data(), dm, g_lm_head, dm, nthreads);
    std::vector<float> dy(n), d(n), dmo(n), dh(n), da(n), dxa(n), d_act(nh), d_gate(nh), d_up(nh), t1(n);
    oracle_sgemm_nn(rows, dm, V, d_logits, V, lm_head, dm, dy.data(), dm, nthreads);
    oracle_rmsnorm_backward(dy.data(), yf.data(), rf.data(), final_norm, d.data(), g_final_norm, rows, dm);
    for (int i = n_layers - 1; i >= 0; --i) {
        const float* const* p = layers + (size_t)i * kLayerParams;
        float* const* g = g_layers + (size_t)i * kLayerParams;
        oracle_rmsnorm_backward(d.data(), ypf[i].data(), rpf[i].data(), p[10], dmo.data(), g[10], rows, dm);
        oracle_sgemm_tn_acc(dm, hid, rows, dmo.data(), dm, act[i].data(), hid, g[9], hid, nthreads);
        oracle_sgemm_nn(rows, hid, dm, dmo.data(), dm, p[9], hid, d_act.data(), hid, nthreads);
        for (size_t j = 0; j < nh; ++j) {
            const float ga = gate[i][j], sig = 1.0f / (1.0f + std::exp(-ga));
            d_up[j] = d_act[j] * (ga * sig);
            d_gate[j] = d_act[j] * up[i][j] * sig * (1.0f + ga * (1.0f - sig));
        }
        oracle_sgemm_tn_acc(hid, dm, rows, d_gate.data(), hid, h[i].data(), dm, g[7], dm, nthreads);
        oracle_sgemm_tn_acc(hid, dm, rows, d_up.data(), hid, h[i].data(), dm, g[8], dm, nthreads);
        oracle_sgemm_nn(rows, dm, hid, d_gate.data(), hid, p[7], dm, dh.data(), dm, nthreads);
        oracle_sgemm_nn(rows, dm, hid, d_up.data(), hid, p[8], dm, t1.data(), dm, nthreads);
        for (size_t j = 0; j < n; ++j) dh[j] += t1[j] + d[j];
        oracle_rmsnorm_backward(dh.data(), ypa[i].data(), rpa[i].data(), p[6], da.data(), g[6], rows, dm);
        oracle_attention_layer_backward(xin[i].data(), p[0], p[1], p[2], p[3], p[4], p[5], sin_t.data(),
                                        cos_t.data(), da.data(), dxa.data(), g[0], g[1], g[2], g[3], g[4], g[5], B, T,
                                        H, 128, eps, nthreads);
        for (size_t j = 0; j < n; ++j) d[j] = dxa[j] + dh[j];
    }
    for (int r = 0; r < rows; ++r) {
        float* dst = g_embed + (int64_t)tokens[r] * dm;
        for (int c = 0; c < dm; ++c) dst[c] += d[(size_t)r * dm + c];
    }
}

}  // extern "C"
