// Process-wide default context of the C++ drop-in wrappers (device 0), created
// on first use and destroyed at exit, plus status-to-exception conversion.
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

inline dt_ctx* default_context() {
    struct Holder {
        dt_ctx* ctx = nullptr;
        ~Holder() {
            if (ctx) dt_ctx_destroy(ctx);
        }
    };
    static Holder h;
    if (!h.ctx) throw_if_error(dt_ctx_create(0, &h.ctx));
    return h.ctx;
}

}  // namespace dt
