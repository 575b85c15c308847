// Shared host/device helpers for the gfx950 library libtbhip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <string>

#include "../../include/tbhip.h"

namespace tb {

// Records the message of the last failing call on this thread and returns code.
int fail(int code, const std::string &msg);

// A stream's device scratch, held by one op while it enqueues its kernels.
struct WsLease {
    std::unique_lock<std::mutex> lock;
    void *ptr = nullptr;
};

// The scratch of stream `st` on the current device, at least `bytes` long.
// One buffer per (device, stream): ops on different streams never share
// scratch, and ops that share a stream are stream-ordered -- the lease keeps a
// second thread on the same stream from interleaving its enqueue.  The buffer
// grows geometrically; a replaced buffer is never freed while the process
// lives (a graph captured earlier may still read it), and growth never
// synchronizes, so it is legal during stream capture.
int workspace(size_t bytes, hipStream_t st, WsLease &out);

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
