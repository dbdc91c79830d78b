// Shared host-side helpers: error recording and HIP status checks.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <string>

#include "gaje_hip.h"

namespace gaje {

// Records `code` with a printf-style message as this thread's last error
// (returned by gaje_hip_last_error) and returns `code`.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

}  // namespace gaje

#define GAJE_HIP_CHECK(expr)                                                                  \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess)                                                                 \
            return ::gaje::set_error(GAJE_ERR_HIP, "%s failed: %s", #expr,                    \
                                     hipGetErrorString(e_));                                  \
    } while (0)

#define GAJE_TRY(expr)                                                                        \
    do {                                                                                      \
        int rc_ = (expr);                                                                     \
        if (rc_ != GAJE_OK) return rc_;                                                       \
    } while (0)
