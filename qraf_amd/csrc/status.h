// status.h -- status codes and the calling thread's last-error text, shared by
// the HIP sources and the plain C++ host sources (no HIP dependency).
#pragma once

#include "../../include/qraf_hip.h"

namespace qraf_hip {

// Sets the calling thread's last-error string and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

#define QH_REQUIRE(cond, code, ...)                                  \
    do {                                                             \
        if (!(cond)) return ::qraf_hip::set_error(code, __VA_ARGS__); \
    } while (0)

// Propagates a failed status (the error text is already set).
#define QH_TRY(expr)                        \
    do {                                    \
        int rc_ = (expr);                   \
        if (rc_ != QRAF_HIP_OK) return rc_; \
    } while (0)

}  // namespace qraf_hip
