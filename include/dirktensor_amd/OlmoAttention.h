// Drop-in for the reference's class OlmoAttention (OlmoAttention.h:10-42) on
// the HIP path. The constructor reads the same per-layer .npy files
// (OlmoAttention.cpp:39-53) and keeps the weights on the GPU; forward takes and
// returns host tensors [batch, seq, d_model] like the reference
// (OlmoAttention.cpp:56-108), computing in fp32 exact mode. As in the
// reference, forward keeps what backward needs (OlmoAttention.h:28-38), here in
// device memory; backward, step and zero_grad follow OlmoAttention.cpp:193-330.
#pragma once

#include <string>

#include "../dirktensor_amd.h"
#include "context.h"
#include "tensor.h"

class OlmoAttention {
public:
    OlmoAttention(const std::string& folder, unsigned int index) {
        dt::throw_if_error(dt_attn_layer_load(dt::default_context(), folder.c_str(), index, &m_layer));
    }
    ~OlmoAttention() {
        if (m_layer) dt_attn_layer_destroy(m_layer);
    }
    OlmoAttention(const OlmoAttention&) = delete;
    OlmoAttention& operator=(const OlmoAttention&) = delete;
    OlmoAttention(OlmoAttention&& o) noexcept : m_layer(o.m_layer) { o.m_layer = nullptr; }

    DT_TENSOR_TEMPLATE<float, 3> forward(const DT_TENSOR_TEMPLATE<float, 3>& input) {
        const int B = (int)input.shape(0), T = (int)input.shape(1);
        auto out = DT_TENSOR_TEMPLATE<float, 3>::from_shape({input.shape(0), input.shape(1), input.shape(2)});
        dt::throw_if_error(dt_attn_layer_fwd(m_layer, input.data(), out.data(), B, T, nullptr, DT_FP32_EXACT,
                                             DT_MEM_HOST, 1, nullptr));
        return out;
    }

    DT_TENSOR_TEMPLATE<float, 3> backward(const DT_TENSOR_TEMPLATE<float, 3>& d_output) {
        auto d_input = DT_TENSOR_TEMPLATE<float, 3>::from_shape({d_output.shape(0), d_output.shape(1), d_output.shape(2)});
        dt::throw_if_error(dt_attn_layer_bwd(m_layer, d_output.data(), d_input.data(), (int)d_output.shape(0),
                                             (int)d_output.shape(1), DT_MEM_HOST, nullptr));
        return d_input;
    }
    void step(float lr) {
        dt::throw_if_error(dt_attn_layer_step(m_layer, lr, nullptr));
        dt::throw_if_error(dt_attn_layer_get_weights(m_layer, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                                     DT_MEM_HOST, nullptr));  // synchronises, like the reference
    }
    void zero_grad() {
        dt::throw_if_error(dt_attn_layer_zero_grad(m_layer, nullptr));
        dt::throw_if_error(dt_attn_layer_get_grads(m_layer, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                                   DT_MEM_HOST, nullptr));
    }

private:
    dt_attn_layer* m_layer = nullptr;
};
