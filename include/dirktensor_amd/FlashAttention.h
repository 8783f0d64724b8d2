// Drop-in for the reference's FlashAttention.h (FlashAttention.h:1-43) on the
// HIP path: same names, argument order, defaults and value semantics (inputs by
// const reference, results as freshly allocated tensors). Tensors live in host
// memory; each call copies to the GPU, runs the fp32 exact-mode kernel and
// copies back (DT_MEM_HOST). Errors throw std::runtime_error.
#pragma once

#include <string>

#include "../dirktensor_amd.h"
#include "context.h"
#include "tensor.h"

// FlashAttention.h:6-10
struct FlashAttentionResult {
    DT_TENSOR_TEMPLATE<float, 4> output;     // (batch, seq, n_heads, head_dim)
    DT_TENSOR_TEMPLATE<float, 3> softmax_m;  // (batch, seq, n_heads)
    DT_TENSOR_TEMPLATE<float, 3> softmax_l;  // (batch, seq, n_heads)
};

// FlashAttention.h:27-31
struct FlashAttentionGradients {
    DT_TENSOR_TEMPLATE<float, 4> d_Q;
    DT_TENSOR_TEMPLATE<float, 4> d_K;
    DT_TENSOR_TEMPLATE<float, 4> d_V;
};

// FlashAttention.h:15-21
inline FlashAttentionResult flash_attention_forward(const DT_TENSOR_TEMPLATE<float, 4>& Q,
                                                    const DT_TENSOR_TEMPLATE<float, 4>& K,
                                                    const DT_TENSOR_TEMPLATE<float, 4>& V, float scale,
                                                    bool causal = true) {
    for (int d = 0; d < 4; ++d)
        if (K.shape(d) != Q.shape(d) || V.shape(d) != Q.shape(d))
            throw std::runtime_error("flash_attention_forward: Q, K, V must have the same shape");
    const int B = (int)Q.shape(0), T = (int)Q.shape(1), H = (int)Q.shape(2), D = (int)Q.shape(3);
    if (D != DT_HEAD_DIM)
        throw std::runtime_error("flash_attention_forward: head_dim " + std::to_string(D) + " != " +
                                 std::to_string(DT_HEAD_DIM));
    if (T < 1 || T > DT_MAX_SEQ_LEN || B < 1 || H < 1)
        throw std::runtime_error("flash_attention_forward: need 1 <= T <= " + std::to_string(DT_MAX_SEQ_LEN) +
                                 ", B >= 1, H >= 1");
    FlashAttentionResult r;
    r.output = DT_TENSOR_TEMPLATE<float, 4>::from_shape({(size_t)B, (size_t)T, (size_t)H, (size_t)D});
    r.softmax_m = DT_TENSOR_TEMPLATE<float, 3>::from_shape({(size_t)B, (size_t)T, (size_t)H});
    r.softmax_l = DT_TENSOR_TEMPLATE<float, 3>::from_shape({(size_t)B, (size_t)T, (size_t)H});
    dt::throw_if_error(dt_flash_attn_fwd(dt::default_context(), Q.data(), K.data(), V.data(), r.output.data(),
                                         r.softmax_m.data(), r.softmax_l.data(), B, T, H, D, scale, causal ? 1 : 0,
                                         nullptr, DT_FP32_EXACT, DT_MEM_HOST, nullptr));
    return r;
}

// FlashAttention.h:33-43
inline FlashAttentionGradients flash_attention_backward(
    const DT_TENSOR_TEMPLATE<float, 4>& d_output, const DT_TENSOR_TEMPLATE<float, 4>& output,
    const DT_TENSOR_TEMPLATE<float, 3>& softmax_m, const DT_TENSOR_TEMPLATE<float, 3>& softmax_l,
    const DT_TENSOR_TEMPLATE<float, 4>& Q, const DT_TENSOR_TEMPLATE<float, 4>& K,
    const DT_TENSOR_TEMPLATE<float, 4>& V, float scale, bool causal = true) {
    for (int d = 0; d < 4; ++d)
        if (K.shape(d) != Q.shape(d) || V.shape(d) != Q.shape(d) || output.shape(d) != Q.shape(d) ||
            d_output.shape(d) != Q.shape(d))
            throw std::runtime_error("flash_attention_backward: d_output, output, Q, K, V must have the same shape");
    for (int d = 0; d < 3; ++d)
        if (softmax_m.shape(d) != Q.shape(d) || softmax_l.shape(d) != Q.shape(d))
            throw std::runtime_error("flash_attention_backward: softmax_m and softmax_l must be [B, T, H]");
    const int B = (int)Q.shape(0), T = (int)Q.shape(1), H = (int)Q.shape(2), D = (int)Q.shape(3);
    if (D != DT_HEAD_DIM)
        throw std::runtime_error("flash_attention_backward: head_dim " + std::to_string(D) + " != " +
                                 std::to_string(DT_HEAD_DIM));
    if (T < 1 || T > DT_MAX_SEQ_LEN || B < 1 || H < 1)
        throw std::runtime_error("flash_attention_backward: need 1 <= T <= " + std::to_string(DT_MAX_SEQ_LEN) +
                                 ", B >= 1, H >= 1");
    FlashAttentionGradients g;
    g.d_Q = DT_TENSOR_TEMPLATE<float, 4>::from_shape({(size_t)B, (size_t)T, (size_t)H, (size_t)D});
    g.d_K = DT_TENSOR_TEMPLATE<float, 4>::from_shape({(size_t)B, (size_t)T, (size_t)H, (size_t)D});
    g.d_V = DT_TENSOR_TEMPLATE<float, 4>::from_shape({(size_t)B, (size_t)T, (size_t)H, (size_t)D});
    dt::throw_if_error(dt_flash_attn_bwd(dt::default_context(), d_output.data(), output.data(), softmax_m.data(),
                                         softmax_l.data(), Q.data(), K.data(), V.data(), g.d_Q.data(), g.d_K.data(),
                                         g.d_V.data(), B, T, H, D, scale, causal ? 1 : 0, DT_FP32_EXACT, DT_MEM_HOST,
                                         nullptr));
    return g;
}
