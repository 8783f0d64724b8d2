// Drop-in for the reference's class OlmoAttention (OlmoAttention.h:10-42) on
// the HIP path. The constructor reads the same per-layer .npy files
// (OlmoAttention.cpp:39-53) and keeps the weights on the GPU; forward takes and
// returns host tensors [batch, seq, d_model] like the reference
// (OlmoAttention.cpp:56-108), computing in fp32 exact mode. backward, step and
// zero_grad throw: the GPU path is forward-only.
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
                                             DT_MEM_HOST, nullptr));
        return out;
    }

    DT_TENSOR_TEMPLATE<float, 3> backward(const DT_TENSOR_TEMPLATE<float, 3>& d_output) {
        DT_TENSOR_TEMPLATE<float, 3> d_input;
        dt::throw_if_error(dt_attn_layer_bwd(m_layer, d_output.data(), d_input.data(), (int)d_output.shape(0),
                                             (int)d_output.shape(1), DT_MEM_HOST, nullptr));
        return d_input;
    }
    void step(float) { throw std::runtime_error("OlmoAttention::step: the GPU path is forward-only"); }
    void zero_grad() { throw std::runtime_error("OlmoAttention::zero_grad: the GPU path is forward-only"); }

private:
    dt_attn_layer* m_layer = nullptr;
};
