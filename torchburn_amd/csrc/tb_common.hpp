// Shared host/device helpers for the gfx950 library libtbhip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/tbhip.h"

namespace tb {

// Records the message of the last failing call on this thread and returns code.
int fail(int code, const std::string &msg);

// The library's device scratch (grow-only, one per device) of at least `bytes`.
int workspace(size_t bytes, void **out);

#define TB_HIP(expr)                                                                   \
    do {                                                                               \
        hipError_t _e = (expr);                                                        \
        if (_e != hipSuccess)                                                          \
            return ::tb::fail(_e == hipErrorOutOfMemory ? TB_ERR_MEMORY : TB_ERR_HIP,  \
                              std::string(#expr) + ": " + hipGetErrorString(_e));      \
    } while (0)

#define TB_REQUIRE(cond, code, msg)                                                    \
    do {                                                                               \
        if (!(cond)) return ::tb::fail((code), (msg));                                 \
    } while (0)

// Launch error check (kernel launches report configuration errors here).
#define TB_LAUNCHED() TB_HIP(hipGetLastError())

}  // namespace tb
