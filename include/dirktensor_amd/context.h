// Process-wide default context of the C++ drop-in wrappers (device 0), created
// on first use and kept for the life of the process, plus status-to-exception
// conversion.
// The reference throws std::runtime_error for failures (main.cpp:40,
// Detokenizer.cpp:44,53); the wrappers do the same with dt_last_error().
#pragma once

#include <stdexcept>
#include <string>

#include "../dirktensor_amd.h"

namespace dt {

inline void throw_if_error(int rc) {
    if (rc != DT_OK) throw std::runtime_error(std::string("dirktensor_amd: ") + dt_last_error());
}

// Created on first use and kept until the process ends, which releases it. It is not destroyed from a static
// destructor: static destructors run in the reverse order of construction, so one registered before the first
// GPU call would run after the statics that the HIP runtime and rocBLAS create lazily on their first use have
// been destroyed, and dt_ctx_destroy (rocblas_destroy_handle, hipFree) would then use freed memory.
inline dt_ctx* default_context() {
    static dt_ctx* const ctx = [] {
        dt_ctx* c = nullptr;
        throw_if_error(dt_ctx_create(0, &c));  // a throw leaves ctx uninitialised: the next call tries again
        return c;
    }();
    return ctx;
}

}  // namespace dt
