// Minimal owning row-major tensor for the C++ drop-in wrappers.
//
// It provides the subset of xt::xtensor<T, N> that the reference's callers use
// on these interfaces: shape(i), shape(), size(), data(), operator()(i, j, ...)
// and the static from_shape({...}). The wrappers are templates over the tensor
// type (DT_TENSOR_TEMPLATE), so a caller holding xtensor can define
// DT_TENSOR_TEMPLATE as xt::xtensor before including them.
#pragma once

#include <array>
#include <cstddef>
#include <initializer_list>
#include <stdexcept>
#include <vector>

namespace dt {

template <class T, std::size_t N>
class tensor {
public:
    using value_type = T;
    using shape_type = std::array<std::size_t, N>;

    tensor() { m_shape.fill(0); }

    static tensor from_shape(const shape_type& s) {
        tensor t;
        t.m_shape = s;
        std::size_t n = 1;
        for (std::size_t d : s) n *= d;
        t.m_data.assign(n, T{});
        return t;
    }
    static tensor from_shape(std::initializer_list<std::size_t> s) {
        if (s.size() != N) throw std::invalid_argument("tensor::from_shape: wrong rank");
        shape_type a{};
        std::size_t i = 0;
        for (std::size_t d : s) a[i++] = d;
        return from_shape(a);
    }

    const shape_type& shape() const { return m_shape; }
    std::size_t shape(std::size_t i) const { return m_shape[i]; }
    std::size_t size() const { return m_data.size(); }
    T* data() { return m_data.data(); }
    const T* data() const { return m_data.data(); }

    template <class... I>
    T& operator()(I... idx) { return m_data[offset(idx...)]; }
    template <class... I>
    const T& operator()(I... idx) const { return m_data[offset(idx...)]; }

private:
    template <class... I>
    std::size_t offset(I... idx) const {
        static_assert(sizeof...(I) == N, "index rank must match tensor rank");
        const std::size_t ix[N] = {static_cast<std::size_t>(idx)...};
        std::size_t o = 0;
        for (std::size_t d = 0; d < N; ++d) o = o * m_shape[d] + ix[d];
        return o;
    }

    shape_type m_shape;
    std::vector<T> m_data;
};

}  // namespace dt

#ifndef DT_TENSOR_TEMPLATE
#define DT_TENSOR_TEMPLATE ::dt::tensor
#endif
